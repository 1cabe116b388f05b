"""fyodor_amd.model: the engine's model description built in Python.

- Every member of the ctypes mirror sits at the offset, and every structure
  has the size, that the C header fyodor_amd/core/llm_internal.h gives it
  (that header is checked against the engine's own by test_boundary.py).
- A resident plan opened on that description through this repository's own
  compute API, against the mock HIP runtime and kernel library, gives the
  logits and KV cache of the engine's scalar reference session over the same
  model written as a GGUF file and loaded by the engine's own loader, within
  the engine's inference-test bounds (backend/tests/test_inference.c:9-33,
  :207-219).
"""
import ctypes
import subprocess

import pytest

from fyodor_amd import F16, Q4_0, Q4_K, Q6_K, Q8_0, Compute
from fyodor_amd import model as fm
from resident_check import bind, plan_against_engine

STRUCTS = {"nya_llm_tensor": fm.Tensor, "nya_llm_layer": fm.Layer, "nya_llm_tokenizer": fm.Tokenizer,
           "nya_llm_mapping": fm.Mapping, "nya_llm_projector": fm.Projector, "nya_llm_context": fm.Context}


def test_ctypes_layout_matches_header(tmp_path):
    from conftest import REPO
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "llm_internal.h"', "int main(void) {"]
    expect = []
    for cname, py in STRUCTS.items():
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        expect.append(f"{cname} {ctypes.sizeof(py)}")
        for field, _ in py._fields_:
            lines.append(f'printf("{cname}.{field} %zu\\n", offsetof({cname}, {field}));')
            expect.append(f"{cname}.{field} {getattr(py, field).offset}")
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c17", f"-I{REPO / 'fyodor_amd/core'}", f"-I{REPO / 'include'}", str(src), "-o",
                    str(exe)], check=True)
    got = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    assert [g for g in got if g] == expect


def test_context_fields_follow_shape():
    shape = fm.LlamaShape()
    m = fm.LlamaModel(shape)
    c = m.context
    assert c.block_count == shape.blocks and c.tokenizer.vocabulary_size == shape.vocabulary
    assert c.tensor_count == 3 + 9 * shape.blocks
    kvd = shape.kv_heads * shape.embedding // shape.heads
    assert [m.layers[b].cache_offset for b in range(shape.blocks)] == [b * kvd for b in range(shape.blocks)]
    assert c.cache_width == shape.blocks * kvd
    assert c.output.contents.name == b"output.weight" and c.output.contents.dimensions[1] == shape.vocabulary


@pytest.fixture()
def mock_rocm(mock_paths, monkeypatch):
    good, _ = mock_paths
    monkeypatch.setenv("NYA_ROCM_HIP_LIBRARY", str(good))
    monkeypatch.setenv("NYA_ROCM_KERNEL_LIBRARY", str(good))
    monkeypatch.delenv("NYA_ROCM_CACHE_MIB", raising=False)


TOKENS = [5, 17, 200, 3, 42, 99, 250, 1, 7, 64]


@pytest.mark.parametrize("types", [
    {"embedding": Q4_K, "output": Q6_K, "attention": Q4_K, "gate_up": Q4_K, "down": Q6_K},
    {"embedding": F16, "output": Q8_0, "attention": Q8_0, "gate_up": Q4_0, "down": Q8_0},
], ids=["k-quants", "q8-q4-f16"])
def test_python_model_plan_matches_engine_session(dropin_library, mock_rocm, tmp_path, types):
    shape = fm.LlamaShape(types=types, context=32)
    plan_against_engine(bind(dropin_library), tmp_path, shape, TOKENS)


def test_gemma_context_matches_the_loader(dropin_library, tmp_path):
    """fyodor_amd.model's Gemma description equals what the engine's loader
    makes of the same model written as GGUF (backend/core/llm_gguf.c:852-990):
    the model fields, and per layer the head shape, window, KV source and
    cache offset, and which tensors are bound."""
    from gguf_model import write_gemma
    from resident_check import Model
    lib = bind(dropin_library)
    for shape in (fm.GemmaShape(), fm.GemmaShape(local=(1, 0, 1, 0), shared_kv_layers=0, global_value=True,
                                                  tied_output=False, output_scales=(), softcap=0.0)):
        path = tmp_path / "gemma.gguf"
        write_gemma(path, shape)
        loaded = Model(lib, path, None)
        try:
            want = fm.Context.from_address(loaded.ptr.value)
            got = fm.GemmaModel(shape).context
            for f in ("embedding_length", "block_count", "is_gemma", "is_assistant", "cache_width", "sliding_window",
                      "final_logit_softcap", "sliding_rope_base", "rope_frequency_base", "norm_epsilon",
                      "expert_count", "per_layer_embedding_length"):
                assert getattr(got, f) == getattr(want, f), f
            assert bool(got.output) and (got.output.contents.name == want.output.contents.name)
            for b in range(shape.blocks):
                g, w = got.layers[b], want.layers[b]
                for f in ("head_count", "kv_head_count", "head_dimension", "hidden_length", "sliding_window",
                          "kv_source", "cache_offset"):
                    assert getattr(g, f) == getattr(w, f), (b, f)
                for f, _ in fm.Layer._fields_:
                    if f in ("head_count", "kv_head_count", "head_dimension", "hidden_length", "expert_hidden_length",
                             "sliding_window", "kv_source", "cache_offset"):
                        continue
                    a, c = getattr(g, f), getattr(w, f)
                    assert bool(a) == bool(c), (b, f)
                    if a:
                        assert a.contents.name == c.contents.name, (b, f)
        finally:
            loaded.close()


def test_python_gemma_plan_matches_engine_session(dropin_library, mock_rocm, tmp_path):
    plan_against_engine(bind(dropin_library), tmp_path, fm.GemmaShape(context=32), TOKENS)


def test_plan_rejects_out_of_range_calls(mock_rocm):
    shape = fm.LlamaShape(context=8)
    compute = Compute("rocm")
    plan = fm.Plan(compute, fm.LlamaModel(shape), 8)
    try:
        with pytest.raises(RuntimeError):
            plan.token(shape.vocabulary, 0)          # token outside the vocabulary
        plan2 = fm.Plan(compute, fm.LlamaModel(shape), 8)
        try:
            with pytest.raises(RuntimeError):
                plan2.token(1, 3)                    # position past the valid prefix
        finally:
            plan2.close()
    finally:
        plan.close()
        compute.close()

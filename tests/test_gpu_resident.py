"""The resident plan on an MI355X: the engine's own inference session and
model loader (backend/core/llm_cpu.c, llm_gguf.c, built from the reference
sources into oracle/_ref/libnya_dropin.so with this repository's provider
registered) run a random-weight LLaMA GGUF (tests/gguf_model.py) with
NYA_COMPUTE=rocm — the whole token forward on the GPU through the gfx950
kernels — and every decode step's logits, the KV cache, and after a reset
prompt chunks (batched through the prefill GEMM and the small-N kernels)
between decode steps, match the engine's scalar reference
session within its own inference-test bounds
(backend/tests/test_inference.c:9-33, :207-219): logits within
5e-4 (1 + |ref|), K/V within 1.5e-4 (1 + |ref|)."""
import ctypes

import pytest

from fyodor_amd import F16, KERNEL_LIBRARY, Q4_0, Q4_K, Q6_K, Q8_0
from gguf_model import GemmaShape, LlamaShape, write, write_gemma
from resident_check import Model, Session, bind, compare, plan_against_engine
from conftest import DROPIN_LIBRARY

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def session_lib():
    """Built beforehand (make -C oracle dropin, where the reference sources
    are); used as built here."""
    if not DROPIN_LIBRARY.exists():
        pytest.skip("oracle/_ref/libnya_dropin.so was not built (it needs the reference sources)")
    return bind(ctypes.CDLL(str(DROPIN_LIBRARY)))


@pytest.fixture()
def rocm_env(monkeypatch):
    monkeypatch.setenv("NYA_ROCM_KERNEL_LIBRARY", str(KERNEL_LIBRARY))
    for v in ("NYA_ROCM_HIP_LIBRARY", "NYA_ROCM_CACHE_MIB", "NYA_INFERENCE_REFERENCE"):
        monkeypatch.delenv(v, raising=False)


TOKENS = [(i * 37 + 11) % 1000 for i in range(40)]


@pytest.mark.parametrize("types", [
    {"embedding": Q4_K, "output": Q6_K, "attention": Q4_K, "gate_up": Q4_K, "down": Q6_K},
    {"embedding": F16, "output": Q8_0, "attention": Q8_0, "gate_up": Q4_0, "down": Q8_0},
    # v and up of other types than q/k and gate: the products run as separate parts.
    {"embedding": Q4_K, "output": Q6_K, "attention": Q4_K, "value": Q6_K, "gate_up": Q4_K, "up": Q8_0, "down": Q6_K},
], ids=["k-quants", "q8-q4-f16", "split-products"])
def test_resident_plan_on_gpu(session_lib, rocm_env, tmp_path, types):
    shape = LlamaShape(embedding=512, heads=8, kv_heads=2, hidden=1024, blocks=3, context=64, vocabulary=1000,
                       types=types, seed=3)
    path = tmp_path / "model.gguf"
    write(path, shape)
    # Prompt chunks of 37 and 13 tokens run the batched forward on the
    # prefill GEMM; 5 on the small-N kernels; single tokens decode.
    out = compare(session_lib, path, shape, "rocm", TOKENS, chunks=(37, 1, 5, 1, 13, 1))
    print(f"resident plan: worst scaled logit error {out['logit']:.3g}, KV {out['kv']:.3g}", flush=True)
    assert out["execution"] == "resident"
    s = out["stats"]
    assert s.kernel_launches > 0 and s.external_matmul_calls > 0 and s.kv_bytes > 0


def test_logits_copy_call_on_gpu(session_lib, rocm_env, tmp_path):
    """A vocabulary of 1001 entries (rows of 4004 bytes, not whole 16-byte
    units for the copy kernel into the mapped staging) takes the logits
    download with a copy call instead; decode and prompt chunks against the
    engine, graphs on."""
    shape = LlamaShape(embedding=512, heads=8, kv_heads=2, hidden=1024, blocks=2, context=64, vocabulary=1001,
                       seed=5)
    path = tmp_path / "model.gguf"
    write(path, shape)
    out = compare(session_lib, path, shape, "rocm", TOKENS[:20], chunks=(9, 1, 1))
    print(f"vocabulary 1001: worst scaled logit error {out['logit']:.3g}, KV {out['kv']:.3g}", flush=True)
    assert out["execution"] == "resident"


# The decoder shapes bench.py times (its resident legs): TinyLlama 1.1B and
# the 8B class, each with its own per-block matrices, head layout,
# vocabulary and Q4_K/Q6_K mix, at fewer blocks than the real models (the
# engine's scalar reference session computes every token on one CPU core;
# every block runs the same kernels). TinyLlama: 4 decode tokens, then a
# 64-token prompt chunk (the prefill GEMM) and a decode step after it; the
# 8B class: 4 decode tokens, a 16-token chunk (8-token launches of the
# small-N kernel) and a decode step.
BENCH_TYPES = {"embedding": Q4_K, "output": Q6_K, "attention": Q4_K, "gate_up": Q4_K, "down": Q6_K}
BENCH_SHAPES = {
    "tinyllama-1.1b": (dict(embedding=2048, heads=32, kv_heads=4, hidden=5632, vocabulary=32000, blocks=2), (64, 1)),
    "llama-8b": (dict(embedding=4096, heads=32, kv_heads=8, hidden=14336, vocabulary=128256, blocks=1), (16, 1)),
}


@pytest.mark.parametrize("name", list(BENCH_SHAPES))
def test_benchmarked_shapes_against_engine(session_lib, rocm_env, tmp_path, name):
    dims, chunks = BENCH_SHAPES[name]
    shape = LlamaShape(**dims, context=sum(chunks) + 8, types=BENCH_TYPES, seed=13)
    path = tmp_path / "model.gguf"
    write(path, shape)
    print(f"{name}: {dims['blocks']} blocks, decode 4 tokens, chunks {chunks}", flush=True)
    out = compare(session_lib, path, shape, "rocm", TOKENS[:4], chunks=chunks)
    print(f"{name}: worst scaled logit error {out['logit']:.3g}, KV {out['kv']:.3g}", flush=True)
    assert out["execution"] == "resident"


def test_long_context_against_engine(session_lib, rocm_env, tmp_path):
    """Decode past 320 cached positions (the split attention: partial
    softmaxes per KV head and position range, then their combination) and a
    20-token run there, against the engine's scalar session."""
    shape = LlamaShape(embedding=512, heads=8, kv_heads=2, hidden=1024, blocks=2, context=440, vocabulary=1000,
                       seed=9)
    path = tmp_path / "model.gguf"
    write(path, shape)
    tokens = [(i * 29 + 7) % shape.vocabulary for i in range(400)]
    out = compare(session_lib, path, shape, "rocm", tokens, chunks=(395, 1, 20, 1))
    print(f"long context: worst scaled logit error {out['logit']:.3g}, KV {out['kv']:.3g}", flush=True)
    assert out["execution"] == "resident"


def test_long_context_graph_replays_match_direct_launches(monkeypatch):
    """Decode tokens past 320 positions replayed as the split-attention graph
    equal direct launches bit for bit, as do the short-context ones before
    them (both graph variants in one plan)."""
    import numpy as np
    from fyodor_amd import Compute
    from fyodor_amd import model as fm
    monkeypatch.setenv("NYA_ROCM_KERNEL_LIBRARY", str(KERNEL_LIBRARY))
    monkeypatch.delenv("NYA_ROCM_HIP_LIBRARY", raising=False)
    shape = fm.LlamaShape(embedding=256, heads=4, kv_heads=2, hidden=8704, blocks=2, context=440, vocabulary=1000,
                          seed=4)
    model = fm.LlamaModel(shape)
    tokens = [(i * 37 + 11) % shape.vocabulary for i in range(420)]

    def decode(graphs: bool):
        monkeypatch.setenv("NYA_ROCM_GRAPHS", "1" if graphs else "0")
        compute = Compute("rocm")
        plan = fm.Plan(compute, model, shape.context)
        rows = []
        try:
            plan.prefill(tokens[:300], 0)
            for i in range(300, 340):
                rows.append(plan.token(tokens[i], i).copy())
            return rows, plan.stats()
        finally:
            plan.close()
            compute.close()

    graphed, g = decode(True)
    direct, d = decode(False)
    assert g["graph_captures"] == 2 and d["graph_replays"] == 0
    assert g["kernel_launches"] == d["kernel_launches"]
    for i, (a, b) in enumerate(zip(graphed, direct)):
        assert np.array_equal(a, b), f"position {300 + i}"


def test_python_model_plan_on_gpu(session_lib, rocm_env, tmp_path):
    """The model description built by fyodor_amd.model (no engine loader),
    planned through this repository's own compute API on the GPU, against
    the engine's reference session of the same model."""
    shape = LlamaShape(embedding=512, heads=8, kv_heads=2, hidden=1024, blocks=3, context=64, vocabulary=1000,
                       seed=5)
    out = plan_against_engine(session_lib, tmp_path, shape, TOKENS[:24])
    print(f"python-built plan: worst scaled logit error {out['logit']:.3g}, KV {out['kv']:.3g}", flush=True)


# Decode shapes for the graph replay check: one where the plan runs the
# separate steps, and one where both one-token fusions engage (512 q|k|v
# rows, two per CU: the normed rotary product; gate|up 17408 rows, past 64
# per CU: the interleaved SwiGLU product).
REPLAY_SHAPES = {"separate-steps": dict(embedding=512, heads=8, kv_heads=2, hidden=1024),
                 "fused-products": dict(embedding=256, heads=4, kv_heads=2, hidden=8704)}


@pytest.mark.parametrize("dims", list(REPLAY_SHAPES.values()), ids=list(REPLAY_SHAPES))
def test_decode_graph_replays_match_direct_launches(monkeypatch, dims):
    """A decode token's launches replayed as a captured HIP graph give the
    same logits, bit for bit, as the same launches issued one by one
    (NYA_ROCM_GRAPHS=0), over many replays of both graphs (with and without
    logits) with eager prompt chunks and host waits between them."""
    import numpy as np
    from fyodor_amd import Compute
    from fyodor_amd import model as fm
    monkeypatch.setenv("NYA_ROCM_KERNEL_LIBRARY", str(KERNEL_LIBRARY))
    monkeypatch.delenv("NYA_ROCM_HIP_LIBRARY", raising=False)
    shape = fm.LlamaShape(**dims, blocks=3, context=64, vocabulary=1000, seed=3)
    if dims["hidden"] == 8704:
        from fyodor_amd.hip import Kernels
        L = Kernels().lib
        up, u, sz = ctypes.c_size_t, ctypes.c_uint, ctypes.c_size_t
        L.nya_hip_matvec_normed_rope.argtypes = [up, u, sz, sz, sz, up, up, up, ctypes.c_float, up, up, up, up, sz,
                                                 sz, sz, sz, up, up, up]
        L.nya_hip_matvec_swiglu.argtypes = [up, u, sz, sz, up, up, up]
        # Both fused entries take this model's products (shape queries).
        assert L.nya_hip_matvec_normed_rope(0, Q4_K, 512, 256, 0, 0, 0, 0, 1e-5, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0,
                                            0) == 0
        assert L.nya_hip_matvec_swiglu(0, Q4_K, 2 * 8704, 256, 0, 0, 0) == 0
    model = fm.LlamaModel(shape)
    tokens = [(i * 37 + 11) % shape.vocabulary for i in range(40)]

    def decode(graphs: bool):
        monkeypatch.setenv("NYA_ROCM_GRAPHS", "1" if graphs else "0")
        compute = Compute("rocm")
        plan = fm.Plan(compute, model, shape.context)
        rows = []
        try:
            rows.append(plan.prefill(tokens[:5], 0).copy())
            for i in range(5, 30):
                if i % 4 == 3:
                    plan.token(tokens[i], i, logits=False)
                else:
                    rows.append(plan.token(tokens[i], i).copy())
            rows.append(plan.prefill(tokens[30:37], 30).copy())
            for i in range(37, 40):
                rows.append(plan.token(tokens[i], i).copy())
            return rows, plan.stats()
        finally:
            plan.close()
            compute.close()

    graphed, g = decode(True)
    direct, d = decode(False)
    assert g["graph_captures"] == 2 and g["graph_replays"] == 28 and d["graph_replays"] == 0
    assert g["kernel_launches"] == d["kernel_launches"] and g["external_matmul_calls"] == d["external_matmul_calls"]
    for i, (a, b) in enumerate(zip(graphed, direct)):
        assert np.array_equal(a, b), f"row {i}"


def test_interleaved_gate_up_on_gpu(session_lib, rocm_env, tmp_path):
    """gate|up above 64 rows per CU: the plan interleaves gate and up rows and
    one-token runs form the gated SiLU in the product's epilogue
    (nya_hip_matvec_swiglu), runs of several through nya_hip_silu_pairs."""
    shape = LlamaShape(hidden=8704, context=24, types={"embedding": Q4_K, "output": Q6_K, "attention": Q4_K,
                                                        "gate_up": Q4_K, "down": Q6_K})
    path = tmp_path / "model.gguf"
    write(path, shape)
    out = compare(session_lib, path, shape, "rocm", [5, 17, 200, 3, 42, 99, 250, 1, 7, 64])
    print(out["logit"], out["kv"], flush=True)
    assert out["execution"] == "resident"


# Gemma 4 text models (the engine's is_gemma branch): local layers with an
# 8..352-position window and global layers of their own head widths, layers
# reading an earlier layer's cache, keys standing in for values, per-head
# q/k/v norms with the half-split rotation, post norms, output scales, the
# GELU gate and a final soft cap.
GEMMA_GPU = {
    "widths-128-256": dict(embedding=512, heads=8, kv_heads=4, width=256, local_width=128, hidden=1024,
                           window=16),
    "widths-256-512": dict(embedding=512, heads=4, kv_heads=2, width=512, local_width=256, hidden=1024,
                           window=20),
    "width-80-q8": dict(embedding=512, heads=8, kv_heads=2, width=128, local_width=80, hidden=1536, window=24,
                        types={"embedding": F16, "output": Q8_0, "attention": Q8_0, "gate_up": Q4_0, "down": Q8_0}),
    "untied-plain": dict(embedding=768, heads=8, kv_heads=2, width=128, local_width=64, hidden=2048, window=12,
                         local=(1, 0, 1, 0), shared_kv_layers=0, global_value=True, tied_output=False,
                         output_scales=(), softcap=0.0),
}


@pytest.mark.parametrize("name", list(GEMMA_GPU))
def test_gemma_plan_on_gpu(session_lib, rocm_env, tmp_path, name):
    shape = GemmaShape(**GEMMA_GPU[name], context=64, vocabulary=1000, seed=7)
    path = tmp_path / "gemma.gguf"
    write_gemma(path, shape)
    print(f"gemma {name}", flush=True)
    out = compare(session_lib, path, shape, "rocm", TOKENS, chunks=(37, 1, 5, 1, 13, 1))
    print(f"gemma {name}: worst scaled logit error {out['logit']:.3g}, KV {out['kv']:.3g}", flush=True)
    assert out["execution"] == "resident"


def test_gemma_long_context_on_gpu(session_lib, rocm_env, tmp_path):
    """Past 320 positions: the global layers' split attention, the local
    layers' split over a 352-position window."""
    shape = GemmaShape(embedding=512, heads=8, kv_heads=4, width=256, local_width=128, hidden=1024, window=352,
                       context=440, vocabulary=1000, seed=8)
    path = tmp_path / "gemma.gguf"
    write_gemma(path, shape)
    tokens = [(i * 29 + 7) % shape.vocabulary for i in range(400)]
    out = compare(session_lib, path, shape, "rocm", tokens, chunks=(395, 1, 20, 1))
    print(f"gemma long context: worst scaled logit error {out['logit']:.3g}, KV {out['kv']:.3g}", flush=True)
    assert out["execution"] == "resident"


def test_gemma_split_512_matches_unsplit_on_gpu(session_lib, rocm_env, tmp_path, monkeypatch):
    """Heads 512 wide (global) and 256 wide (local) past 320 positions: a
    session whose attention splits against one that never splits
    (NYA_ROCM_ATTENTION_SPLIT=0), the same model on the same GPU, every
    decode step's logits and the caches within the engine's bounds. The
    unsplit kernels meet the engine at these widths elsewhere; against the
    engine itself this random 512-wide stack is ill-conditioned at single
    positions before any split (the engine's own reference and optimized CPU
    sessions differ in layer 2's cache by 3.1e-5 to 3.1e-4 there, seed by
    seed), which a direct comparison would test instead of the split."""
    import numpy as np
    from resident_check import check_kv, check_logits, kv_widths
    shape = GemmaShape(embedding=512, heads=4, kv_heads=2, width=512, local_width=256, hidden=1024, window=352,
                       context=440, vocabulary=1000, seed=13)
    path = tmp_path / "gemma.gguf"
    write_gemma(path, shape)
    tokens = [(i * 29 + 7) % shape.vocabulary for i in range(400)]

    def open_session(split: bool):
        if split:
            monkeypatch.delenv("NYA_ROCM_ATTENTION_SPLIT", raising=False)
        else:
            monkeypatch.setenv("NYA_ROCM_ATTENTION_SPLIT", "0")
        model = Model(session_lib, path, "rocm")
        return model, Session(model, shape.context)

    (split_model, split), (plain_model, plain) = open_session(True), open_session(False)
    monkeypatch.delenv("NYA_ROCM_ATTENTION_SPLIT", raising=False)
    try:
        differ, worst = False, 0.0
        for i, t in enumerate(tokens):
            assert split.run([t], True) == 0 and plain.run([t], True) == 0
            a, b = plain.logits(shape.vocabulary), split.logits(shape.vocabulary)
            worst = max(worst, check_logits(a, b, f"decode position {i}"))
            differ |= not np.array_equal(a, b)
        kv = check_kv(plain, split, kv_widths(shape), len(tokens))
        assert split.execution() == plain.execution() == "resident"
        # The split sessions' launches add the combine passes past 320 positions.
        assert split.stats().kernel_launches > plain.stats().kernel_launches
        assert differ
        print(f"gemma 512 split vs unsplit: worst scaled logit error {worst:.3g}, KV {kv:.3g}", flush=True)
    finally:
        split.close()
        plain.close()
        split_model.close()
        plain_model.close()


def test_gemma_graph_replays_match_direct_launches(session_lib, rocm_env, tmp_path, monkeypatch):
    """A Gemma decode token replayed as a captured graph (the embedding
    scale, head norms, post norms, GELU gate and soft cap among its
    launches) gives the logits of direct launches bit for bit."""
    import numpy as np
    shape = GemmaShape(**GEMMA_GPU["widths-128-256"], context=64, vocabulary=1000, seed=9)
    path = tmp_path / "gemma.gguf"
    write_gemma(path, shape)

    def run(graphs: bool):
        monkeypatch.setenv("NYA_ROCM_GRAPHS", "1" if graphs else "0")
        model = Model(session_lib, path, "rocm")
        session = Session(model, shape.context)
        rows = []
        try:
            assert session.run(TOKENS[:5], False) == 0
            rows.append(session.logits(shape.vocabulary))
            for t in TOKENS[5:30]:
                assert session.run([t], True) == 0
                rows.append(session.logits(shape.vocabulary))
            assert session.execution() == "resident"
            return rows, session.stats()
        finally:
            session.close()
            model.close()

    graphed, g = run(True)
    direct, d = run(False)
    assert g.graph_replays > 0 and d.graph_replays == 0
    assert g.kernel_launches == d.kernel_launches
    for i, (a, b) in enumerate(zip(graphed, direct)):
        assert np.array_equal(a, b), f"row {i}"

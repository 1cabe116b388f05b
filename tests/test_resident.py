"""The resident plan on the CPU, through the engine's own session and model
loader (backend/core/llm_cpu.c, llm_gguf.c built from the reference sources
with this repository's provider registered), against the mock HIP runtime
and kernel library (tests/mock/mock_hip.c, whose resident steps compute in
the engine's order on the host):

- a random-weight LLaMA GGUF (tests/gguf_model.py) loads, the session runs
  "resident" on the rocm provider, and every decode step's logits and the KV
  cache match the engine's scalar reference session within the engine's own
  inference-test bounds (backend/tests/test_inference.c:9-33, :207-219);
  after a reset, prefill chunks (the plan's prefill) between decode steps
  match too;
- a kernel library without the resident steps declines the plan, and the
  engine then runs its reference path (backend/core/llm_cpu.c:235-242) with
  the same logits.
The same comparison runs on an MI355X in tests/test_gpu_resident.py."""
import subprocess

import pytest

from fyodor_amd import Q4_0, Q4_K, Q6_K, Q8_0, F16
from gguf_model import GemmaShape, LlamaShape, write, write_gemma
from resident_check import bind, compare

TOKENS = [5, 17, 200, 3, 42, 99, 250, 1, 7, 64, 128, 33]


@pytest.fixture()
def session_lib(dropin_library, mock_paths, monkeypatch):
    good, _ = mock_paths
    monkeypatch.setenv("NYA_ROCM_HIP_LIBRARY", str(good))
    monkeypatch.setenv("NYA_ROCM_KERNEL_LIBRARY", str(good))
    monkeypatch.delenv("NYA_ROCM_CACHE_MIB", raising=False)
    monkeypatch.delenv("NYA_INFERENCE_REFERENCE", raising=False)
    return bind(dropin_library)


@pytest.mark.parametrize("types", [
    {"embedding": Q4_K, "output": Q6_K, "attention": Q4_K, "gate_up": Q4_K, "down": Q6_K},
    {"embedding": F16, "output": Q8_0, "attention": Q8_0, "gate_up": Q4_0, "down": Q8_0},
    {"embedding": Q4_K, "output": Q6_K, "attention": Q4_K, "value": Q6_K, "gate_up": Q4_K, "up": Q8_0, "down": Q6_K},
], ids=["k-quants", "q8-q4-f16", "split-products"])
def test_resident_plan_matches_reference_session(session_lib, tmp_path, types):
    shape = LlamaShape(types=types, context=32)
    path = tmp_path / "model.gguf"
    write(path, shape)
    out = compare(session_lib, path, shape, "rocm", TOKENS)
    assert out["execution"] == "resident"
    s = out["stats"]
    assert s.kernel_launches > 0 and s.external_matmul_calls > 0 and s.kv_bytes > 0 and s.weights_bytes > 0


def test_long_context_split_attention(session_lib, tmp_path, monkeypatch):
    """Past 320 cached positions decode tokens and runs of up to 33 tokens
    take the split attention (nya_hip_attention_split: partial softmaxes
    through the plan's scratch, then their combination); logits and KV still
    match the engine's reference session, and the split adds one launch per
    block and run (NYA_ROCM_ATTENTION_SPLIT=0 keeps every run unsplit)."""
    shape = LlamaShape(context=420)
    path = tmp_path / "model.gguf"
    write(path, shape)
    tokens = [(i * 29 + 7) % shape.vocabulary for i in range(390)]
    split = compare(session_lib, path, shape, "rocm", tokens, chunks=(390, 1, 20, 1))
    assert split["execution"] == "resident"
    monkeypatch.setenv("NYA_ROCM_ATTENTION_SPLIT", "0")
    plain = compare(session_lib, path, shape, "rocm", tokens, chunks=(390, 1, 20, 1))
    # The decode tokens at positions 320..389, then (after the reset and the
    # unsplit 390-token run) the decode at 390, the 20-token run and the
    # decode after it: one more launch per block each.
    assert split["stats"].kernel_launches - plain["stats"].kernel_launches == shape.blocks * (70 + 3)


def test_plan_declined_without_resident_steps(session_lib, tmp_path, monkeypatch):
    lib_dir = tmp_path / "mock"
    lib_dir.mkdir()
    plain = lib_dir / "libnya_mock_plain.so"
    from conftest import REPO
    src = [str(REPO / "tests/mock/mock_hip.c"), str(REPO / "oracle/quant_oracle.c")]
    subprocess.run(["gcc", "-std=c17", "-O1", "-fPIC", "-shared", "-D_POSIX_C_SOURCE=200809L",
                    "-Dnya_hip_rope_qkv=nya_mock_unused_rope", *src, "-o", str(plain), "-lm", "-lpthread"], check=True)
    monkeypatch.setenv("NYA_ROCM_KERNEL_LIBRARY", str(plain))
    shape = LlamaShape(context=16)
    path = tmp_path / "model.gguf"
    write(path, shape)
    out = compare(session_lib, path, shape, "rocm", TOKENS[:6])
    assert out["execution"] == "cpu-reference"


def test_plan_declined_when_its_workspace_exceeds_the_budget(session_lib, tmp_path, monkeypatch):
    """The budget check counts the kernels' workspace (sized for the plan's
    prompt chunks) before allocating anything: a workspace past the budget
    declines the plan, and the engine runs its reference path."""
    shape = LlamaShape(context=16)
    path = tmp_path / "model.gguf"
    write(path, shape)
    # What the plan needs without a workspace, then a budget 4 MiB above it.
    monkeypatch.setenv("MOCK_HIP_GEMM_WORKSPACE", "0")
    out = compare(session_lib, path, shape, "rocm", TOKENS[:4])
    assert out["execution"] == "resident"
    s = out["stats"]
    mib = (s.weights_bytes + s.kv_bytes + s.scratch_bytes + (1 << 20) - 1 >> 20) + 4
    monkeypatch.setenv("NYA_ROCM_CACHE_MIB", str(mib))
    monkeypatch.setenv("MOCK_HIP_GEMM_WORKSPACE", str(2 << 20))
    assert compare(session_lib, path, shape, "rocm", TOKENS[:4])["execution"] == "resident"
    # 8 MiB of workspace would still allocate on the stand-in, but it is past
    # the budget: declined before any upload.
    monkeypatch.setenv("MOCK_HIP_GEMM_WORKSPACE", str(8 << 20))
    assert compare(session_lib, path, shape, "rocm", TOKENS[:4])["execution"] == "cpu-reference"


def mock_without(tmp_path, entries):
    """The mock kernel library built with `entries` renamed away."""
    lib_dir = tmp_path / "mock"
    lib_dir.mkdir()
    plain = lib_dir / "libnya_mock_without.so"
    from conftest import REPO
    src = [str(REPO / "tests/mock/mock_hip.c"), str(REPO / "oracle/quant_oracle.c")]
    subprocess.run(["gcc", "-std=c17", "-O1", "-fPIC", "-shared", "-D_POSIX_C_SOURCE=200809L",
                    *[f"-D{e}=nya_mock_unused_{e}" for e in entries], *src, "-o", str(plain), "-lm", "-lpthread"],
                   check=True)
    return plain


@pytest.mark.parametrize("family", ["llama", "gemma"])
def test_logits_written_into_mapped_staging(session_lib, mock_paths, tmp_path, monkeypatch, family):
    """With the runtime's device address of mapped pinned memory and the
    kernel library's copy, each run's logits reach the host without a copy
    call: the vocabulary product writes the mapped staging itself (LLaMA),
    or one copy launch follows Gemma's soft cap. A kernel library without
    nya_hip_copy leaves the plan downloading them with a copy call. The
    logits meet the engine's either way."""
    import ctypes
    runtime = ctypes.CDLL(str(mock_paths[0]))   # the HIP runtime in both runs
    if family == "gemma":
        shape = GemmaShape(context=16)   # the default test model: a soft cap of 30
        assert shape.softcap > 0
        path = tmp_path / "gemma.gguf"
        write_gemma(path, shape)
    else:
        shape = LlamaShape(context=16)
        path = tmp_path / "model.gguf"
        write(path, shape)
    before = runtime.nya_mock_d2h_copies()
    mapped = compare(session_lib, path, shape, "rocm", TOKENS[:6])
    mapped_d2h = runtime.nya_mock_d2h_copies() - before
    monkeypatch.setenv("NYA_ROCM_KERNEL_LIBRARY", str(mock_without(tmp_path, ("nya_hip_copy",))))
    before = runtime.nya_mock_d2h_copies()
    copied = compare(session_lib, path, shape, "rocm", TOKENS[:6])
    copied_d2h = runtime.nya_mock_d2h_copies() - before
    assert mapped["execution"] == copied["execution"] == "resident"
    s, c = mapped["stats"], copied["stats"]
    assert s.downloads == c.downloads > 0
    # Runs that return logits: six decode tokens, then the five runs of the
    # chunk phase (compare's default chunks); each is a copy call fewer.
    runs = 6 + 5
    assert copied_d2h - mapped_d2h == runs
    assert s.kernel_launches - c.kernel_launches == (runs if family == "gemma" else 0)


def test_logits_downloaded_when_the_row_is_not_whole_16_bytes(session_lib, tmp_path, monkeypatch):
    """A vocabulary of 1001 entries (4004 bytes a row, not a multiple of the
    copy kernel's 16) keeps the copy call: the same launches as a kernel
    library without nya_hip_copy, and the engine's logits."""
    shape = LlamaShape(context=16, vocabulary=1001)
    path = tmp_path / "model.gguf"
    write(path, shape)
    plain = compare(session_lib, path, shape, "rocm", TOKENS[:6])
    monkeypatch.setenv("NYA_ROCM_KERNEL_LIBRARY", str(mock_without(tmp_path, ("nya_hip_copy",))))
    copied = compare(session_lib, path, shape, "rocm", TOKENS[:6])
    assert plain["execution"] == copied["execution"] == "resident"
    assert plain["stats"].kernel_launches == copied["stats"].kernel_launches


@pytest.mark.parametrize("entries,extra", [(("nya_hip_matvec_gated",), 1), (("nya_hip_matvec_normed_rope",), 1),
                                           (("nya_hip_matvec_normed", "nya_hip_matvec_normed_rope"), 2)])
def test_plan_without_fused_step(session_lib, tmp_path, monkeypatch, entries, extra):
    """A kernel library without one of the optional one-token fusions
    (nya_hip_matvec_gated: the gated SiLU in the down product;
    nya_hip_matvec_normed: the attention norm in the q|k|v product;
    nya_hip_matvec_normed_rope: the rotary step in its epilogue) keeps the
    resident plan: the steps run apart, with `extra` more launches per block
    and decode token."""
    plain = mock_without(tmp_path, entries)
    shape = LlamaShape(context=16)
    path = tmp_path / "model.gguf"
    write(path, shape)
    launches = {}
    for name, lib in (("fused", None), ("unfused", plain)):
        if lib is not None:
            monkeypatch.setenv("NYA_ROCM_KERNEL_LIBRARY", str(lib))
        out = compare(session_lib, path, shape, "rocm", TOKENS[:6])
        assert out["execution"] == "resident"
        launches[name] = out["stats"].kernel_launches
    # compare() runs 6 decode tokens, then chunks (5, 1, 1, 7, 1): 9 one-token runs.
    assert launches["unfused"] - launches["fused"] == 9 * extra * shape.blocks, launches


def test_interleaved_gate_up(session_lib, tmp_path, monkeypatch):
    """A feed-forward wide enough for the library's one-token SwiGLU product
    (gate|up above 64 rows per CU): the plan lays gate and up out in 16-row
    blocks; one-token runs take nya_hip_matvec_residual (the attention
    output product with the residual add and the feed-forward norm's
    inputs) and nya_hip_matvec_swiglu_scaled (from a library without the
    pair: the output product, the norm step and nya_hip_matvec_swiglu, one
    launch more per block and token), runs of several nya_hip_silu_pairs (no
    separate SiLU step); logits and cache still match the engine's reference
    session either way."""
    shape = LlamaShape(hidden=8704, context=16, types={"embedding": Q4_K, "output": Q6_K, "attention": Q4_K,
                                                        "gate_up": Q4_K, "down": Q6_K})
    path = tmp_path / "model.gguf"
    write(path, shape)
    launches = {}
    for name, lib in (("fused", None), ("unfused", mock_without(tmp_path, ("nya_hip_matvec_residual", "nya_hip_matvec_swiglu_scaled")))):
        if lib is not None:
            monkeypatch.setenv("NYA_ROCM_KERNEL_LIBRARY", str(lib))
        out = compare(session_lib, path, shape, "rocm", TOKENS[:6])
        assert out["execution"] == "resident"
        launches[name] = out["stats"].kernel_launches
    # 6 decode tokens, then chunks (5, 1, 1, 7, 1): 9 one-token runs.
    assert launches["unfused"] - launches["fused"] == 9 * shape.blocks, launches


GEMMA_VARIANTS = {
    # Tied output, global layers storing the key as the value, two layers
    # reading earlier caches, output scales, a soft cap, an 8-position window.
    "tied-shared": GemmaShape(),
    # An output matrix of its own, value matrices everywhere, no sharing,
    # no output scales and no soft cap.
    "untied-plain": GemmaShape(local=(1, 0, 1, 0), shared_kv_layers=0, global_value=True, tied_output=False,
                               output_scales=(), softcap=0.0),
    # Other weight types, local heads as wide as the global ones.
    "q8-q4-f16": GemmaShape(local_width=128, types={"embedding": F16, "output": Q8_0, "attention": Q8_0,
                                                    "gate_up": Q4_0, "down": Q8_0}),
}


@pytest.mark.parametrize("variant", list(GEMMA_VARIANTS))
def test_gemma_plan_matches_reference_session(session_lib, tmp_path, variant):
    """A Gemma 4 text model (tests/gguf_model.py GemmaShape: the engine's
    is_gemma branch, backend/core/llm_cpu.c:452-566) runs resident: every
    decode step's logits and the KV caches of every layer (a shared layer
    reads its source's) match the engine's reference session, through
    windows shorter than the sequence and prompt chunks."""
    shape = GEMMA_VARIANTS[variant]
    path = tmp_path / "gemma.gguf"
    write_gemma(path, shape)
    out = compare(session_lib, path, shape, "rocm", TOKENS)
    assert out["execution"] == "resident"
    assert out["stats"].kernel_launches > 0


def test_gemma_long_context_split(session_lib, tmp_path):
    """Past 320 positions the global layers take the split attention and the
    local layers (a 352-position window, also past the split threshold) split
    only the window: logits and KV still match the engine."""
    shape = GemmaShape(context=420, window=352)
    path = tmp_path / "gemma.gguf"
    write_gemma(path, shape)
    tokens = [(i * 29 + 7) % shape.vocabulary for i in range(390)]
    out = compare(session_lib, path, shape, "rocm", tokens, chunks=(390, 1, 20, 1))
    assert out["execution"] == "resident"


def test_gemma_declined_without_its_steps(session_lib, tmp_path, monkeypatch):
    """A kernel library without the Gemma steps declines a Gemma model (the
    engine runs its reference path, same logits) and still runs LLaMA."""
    plain = mock_without(tmp_path, ("nya_hip_head_norm_rope",))
    monkeypatch.setenv("NYA_ROCM_KERNEL_LIBRARY", str(plain))
    shape = GemmaShape()
    path = tmp_path / "gemma.gguf"
    write_gemma(path, shape)
    assert compare(session_lib, path, shape, "rocm", TOKENS[:4])["execution"] == "cpu-reference"
    llama = LlamaShape(context=16)
    path = tmp_path / "llama.gguf"
    write(path, llama)
    assert compare(session_lib, path, llama, "rocm", TOKENS[:4])["execution"] == "resident"


def test_gemma_interleaved_gate_up(session_lib, tmp_path, monkeypatch):
    """A Gemma feed-forward wide enough for the library's one-token gate|up
    product (gate|up above 32 rows per CU): the plan interleaves gate and up
    rows, one-token runs form the GELU gate in the product
    (nya_hip_matvec_geglu), runs of several through nya_hip_gelu_pairs;
    logits and cache still match the engine; from a library without the
    product, one launch more per block and one-token run."""
    shape = GemmaShape(hidden=8704, context=16)
    path = tmp_path / "gemma.gguf"
    write_gemma(path, shape)
    launches = {}
    for name, lib in (("fused", None), ("unfused", mock_without(tmp_path, ("nya_hip_matvec_geglu",)))):
        if lib is not None:
            monkeypatch.setenv("NYA_ROCM_KERNEL_LIBRARY", str(lib))
        out = compare(session_lib, path, shape, "rocm", TOKENS[:6])
        assert out["execution"] == "resident"
        launches[name] = out["stats"].kernel_launches
    # 6 decode tokens, then chunks (5, 1, 1, 7, 1): 9 one-token runs.
    assert launches["unfused"] - launches["fused"] == 9 * shape.blocks, launches


@pytest.mark.parametrize("hidden", [1024, 8704], ids=["normed", "scaled"])
def test_rotary_products_in_parts(session_lib, tmp_path, monkeypatch, hidden):
    """q|k in Q4_K and v in Q6_K (a Q4_K_M model's value matrices): one-token
    runs take both parts in one rotary launch (nya_hip_matvec_rope_pair; with
    the interleaved gate|up, blocks after the first take its scaled form);
    from a library without it, one rotary product per part
    (nya_hip_matvec_normed_rope / nya_hip_matvec_scaled_rope with the part's
    first row), one launch more per block and one-token run; without the
    rotary product, the norm step, two products and the rotary step, two
    more. Logits and cache match the engine every way."""
    types = {"embedding": Q4_K, "output": Q6_K, "attention": Q4_K, "value": Q6_K, "gate_up": Q4_K, "down": Q6_K}
    shape = LlamaShape(embedding=512, heads=8, kv_heads=8, hidden=hidden, context=16, types=types)
    path = tmp_path / "model.gguf"
    write(path, shape)
    launches = {}
    for name, entries in (("pair", ()), ("parts", ("nya_hip_matvec_rope_pair",)),
                          ("separate", ("nya_hip_matvec_normed_rope",))):
        if entries:
            lib_dir = tmp_path / name
            lib_dir.mkdir()
            monkeypatch.setenv("NYA_ROCM_KERNEL_LIBRARY", str(mock_without(lib_dir, entries)))
        out = compare(session_lib, path, shape, "rocm", TOKENS[:6])
        assert out["execution"] == "resident"
        launches[name] = out["stats"].kernel_launches
    # 6 decode tokens, then chunks (5, 1, 1, 7, 1): 9 one-token runs.
    assert launches["parts"] - launches["pair"] == 9 * shape.blocks, launches
    assert launches["separate"] - launches["parts"] == 2 * 9 * shape.blocks, launches

"""The engine's own benchmark, `fyodor-bench -b rocm` (backend/core/bench_main.c,
built from the reference sources with this repository's provider registered
into oracle/_ref/fyodor-bench), end to end on the CPU against the mock HIP
runtime and kernel library (tests/mock/mock_hip.c).

The checks restate the reference's adapter smoke test
(backend/tests/BenchVendor.cmake:1-21: `-p 8 -n 8 -r 2 --warmup 1 --json`,
backend named as requested, device weights reported, and every result
counting real provider operations rather than a CPU fallback), with one
difference: this provider runs the whole token forward as a resident plan,
so the session reports "resident" where the reference's matmul-only mock
reports "gpu-assisted". The same run on an MI355X, at TinyLlama 1.1B's shape
with pp512 / tg128, is tests/test_gpu_engine_bench.py."""
import json
import subprocess

import pytest

from conftest import REPO
from gguf_model import GemmaShape, LlamaShape, write, write_gemma

BENCH = REPO / "oracle" / "_ref" / "fyodor-bench"


@pytest.fixture(scope="module")
def bench_binary():
    proc = subprocess.run(["make", "-C", str(REPO / "oracle"), "bench"], capture_output=True, text=True)
    if proc.returncode != 0 or not BENCH.exists():
        pytest.skip("reference sources not mounted: fyodor-bench is built from backend/core of the reference tree")
    return BENCH


def run_bench(binary, model, env, *args):
    proc = subprocess.run([str(binary), "-m", str(model), *args, "--json"], capture_output=True, text=True,
                          env=env, timeout=300)
    assert proc.returncode == 0, proc.stderr
    return json.loads(proc.stdout)


def check_contract(out: dict, backend: str, execution: str):
    """backend/tests/BenchVendor.cmake:11-21, for a resident provider."""
    assert out["backend"] == backend and out["execution"] == execution, out
    assert out["device_memory_after"]["weights_bytes"] > 0 and out["device_kv_bytes"] > 0
    assert len(out["results"]) == 2
    for r in out["results"]:
        assert r["tokens_per_second"] > 0
        assert r["kernel_launches"] > 0 and r["external_matmul_calls"] > 0, r
        assert r["downloads"] > 0 and r["synchronizations"] > 0, r
        # A prompt's token ids are uploaded; a decode token's id reaches the
        # device as a kernel argument (no copy).
        assert (r["uploads"] > 0) == r["test"].startswith("pp"), r


def test_engine_bench_on_mock_provider(bench_binary, mock_paths, tmp_path):
    import os
    good, _ = mock_paths
    model = tmp_path / "model.gguf"
    write(model, LlamaShape(context=32))
    env = dict(os.environ, NYA_ROCM_HIP_LIBRARY=str(good), NYA_ROCM_KERNEL_LIBRARY=str(good))
    env.pop("NYA_ROCM_CACHE_MIB", None)
    out = run_bench(bench_binary, model, env, "-b", "rocm", "-p", "8", "-n", "8", "-r", "2", "--warmup", "1")
    check_contract(out, "rocm", "resident")
    assert out["prefill_implementation"] == "native"
    # The same workload on the engine's CPU provider: same schema, no
    # provider operations.
    cpu = run_bench(bench_binary, model, env, "-b", "cpu", "-p", "8", "-n", "8", "-r", "2", "--warmup", "1")
    assert cpu["backend"] == "cpu" and cpu["execution"] == "cpu-optimized"


def test_engine_bench_gemma_on_mock_provider(bench_binary, mock_paths, tmp_path):
    """A Gemma 4 model through the engine's benchmark runs resident too."""
    import os
    good, _ = mock_paths
    model = tmp_path / "gemma.gguf"
    write_gemma(model, GemmaShape(context=32))
    env = dict(os.environ, NYA_ROCM_HIP_LIBRARY=str(good), NYA_ROCM_KERNEL_LIBRARY=str(good))
    env.pop("NYA_ROCM_CACHE_MIB", None)
    out = run_bench(bench_binary, model, env, "-b", "rocm", "-p", "8", "-n", "8", "-r", "2", "--warmup", "1")
    check_contract(out, "rocm", "resident")


def test_engine_bench_declines_unknown_provider(bench_binary, tmp_path):
    model = tmp_path / "model.gguf"
    write(model, LlamaShape(context=32))
    proc = subprocess.run([str(bench_binary), "-m", str(model), "-b", "nonesuch", "-p", "8", "-n", "0"],
                          capture_output=True, text=True, timeout=60)
    assert proc.returncode == 2

"""`fyodor-bench -b rocm` on an MI355X: the engine's own token-throughput
benchmark (backend/core/bench_main.c, built from the reference sources with
this repository's provider registered into oracle/_ref/fyodor-bench) loads a
synthetic LLaMA GGUF through the engine's loader and runs it through the
resident plan on the gfx950 kernels.

- the reference's adapter contract (backend/tests/BenchVendor.cmake:1-21) on
  a small model, as tests/test_engine_bench.py checks it on the mock;
- the reference's published end-to-end workload (backend/README.md:796-803:
  TinyLlama 1.1B, pp512 and tg128) at TinyLlama's shape (embedding 2048, 32
  heads / 4 KV of 64, feed-forward 5632, 22 blocks, vocabulary 32000) with
  Q4_K attention/gate/up and Q6_K down/output, random weights (no model file
  is available offline; every block stores the same bytes). The JSON line is
  written to $FYODOR_ENGINE_BENCH_OUT when that is set."""
import json
import os
import subprocess

import pytest

from conftest import REPO
from fyodor_amd import KERNEL_LIBRARY, Q4_K, Q6_K
from gguf_model import GemmaShape, LlamaShape, write, write_gemma
from test_engine_bench import check_contract

pytestmark = pytest.mark.gpu

BENCH = REPO / "oracle" / "_ref" / "fyodor-bench"


@pytest.fixture(scope="module")
def env():
    if not BENCH.exists():
        pytest.skip("oracle/_ref/fyodor-bench was not built (it needs the reference sources)")
    e = dict(os.environ, NYA_ROCM_KERNEL_LIBRARY=str(KERNEL_LIBRARY))
    for v in ("NYA_ROCM_HIP_LIBRARY", "NYA_ROCM_CACHE_MIB", "NYA_INFERENCE_REFERENCE", "NYA_COMPUTE"):
        e.pop(v, None)
    return e


def run(model, env, *args):
    proc = subprocess.run([str(BENCH), "-m", str(model), "-b", "rocm", *args, "--json"], capture_output=True,
                          text=True, env=env, timeout=600)
    assert proc.returncode == 0, proc.stderr
    return json.loads(proc.stdout)


def test_engine_bench_contract_on_gpu(env, tmp_path):
    model = tmp_path / "model.gguf"
    write(model, LlamaShape(embedding=512, heads=8, kv_heads=2, hidden=1024, blocks=3, context=64, vocabulary=1000))
    out = run(model, env, "-p", "8", "-n", "8", "-r", "2", "--warmup", "1")
    check_contract(out, "rocm", "resident")


def test_engine_bench_gemma_contract_on_gpu(env, tmp_path):
    """A Gemma 4 model (local and global layers, shared KV, soft cap) through
    the engine's benchmark on the GPU: resident, with the contract's
    counters."""
    model = tmp_path / "gemma.gguf"
    write_gemma(model, GemmaShape(embedding=512, heads=8, kv_heads=4, width=256, local_width=128, hidden=1024,
                                  window=16, context=64, vocabulary=1000))
    out = run(model, env, "-p", "8", "-n", "8", "-r", "2", "--warmup", "1")
    check_contract(out, "rocm", "resident")


def test_engine_bench_tinyllama_shape(env, tmp_path):
    shape = LlamaShape(embedding=2048, heads=32, kv_heads=4, hidden=5632, blocks=22, context=1024, vocabulary=32000,
                       types={"embedding": Q4_K, "output": Q6_K, "attention": Q4_K, "gate_up": Q4_K, "down": Q6_K},
                       seed=7)
    model = tmp_path / "tinyllama-shape.gguf"
    write(model, shape, shared_blocks=True)
    out = run(model, env, "-p", "512", "-n", "128", "-r", "3", "--warmup", "1")
    print(json.dumps(out), flush=True)
    if os.environ.get("FYODOR_ENGINE_BENCH_OUT"):
        with open(os.environ["FYODOR_ENGINE_BENCH_OUT"], "w") as f:
            f.write(json.dumps(out) + "\n")
    assert out["backend"] == "rocm" and out["execution"] == "resident"
    assert {r["test"] for r in out["results"]} == {"pp512", "tg128"}
    assert all(r["tokens_per_second"] > 0 and r["external_matmul_calls"] > 0 for r in out["results"])

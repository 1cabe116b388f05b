"""The CPU leg of bench.py (the reference CPU provider, or the C port where
oracle/_ref is not built), run on a reduced shape so that it takes a second."""
import sys
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
import bench  # noqa: E402
from oracle import Oracle  # noqa: E402


def test_host_cpu_names_a_reference_isa():
    host = bench.host_cpu()
    assert isinstance(host["model"], str) and "family" in host["model"]
    # backend/core/cpu_kernels.c:91-100 selects one of these three.
    assert host["isa"] in ("avx512", "avx2", "scalar")
    assert 1 <= host["affinity_cpus"] <= host["online_cpus"]
    assert host["l3_bytes"] >= 0


def test_cpu_baseline_fields(monkeypatch):
    rows, cols = 64, 4096
    # cpu_baseline sets the provider's thread count; restored afterwards.
    monkeypatch.setenv("NYA_CPU_THREADS", "1")
    monkeypatch.setattr(bench, "ROWS", rows)
    monkeypatch.setattr(bench, "COLS", cols)
    w = bench.synth.weights(bench.Q4_K, rows, cols, seed=7)
    x = bench.synth.activations(1, cols, seed=7)[0].copy()
    y = Oracle().matmul(w, bench.Q4_K, x, rows, cols, 1)[0]
    line = bench.cpu_baseline(w, x, y, 0.05)
    assert line["kind"] in ("reference", "port")
    assert line["unit"] == "GB/s" and line["value"] > 0 and line["cores"] >= 1
    assert line["one_thread"]["value"] > 0 and line["one_thread"]["unit"] == "GB/s"
    assert line["affinity"]["value"] > 0 and line["affinity"]["cores"] >= 1
    assert "family" in line["cpu_model"] and line["online_cpus"] >= 1
    assert line["isa"] in ("avx512", "avx2", "scalar")
    # Both CPU paths are within float rounding of the scalar restatement.
    assert line["parity_rel_l2_vs_gpu"] < 1e-5

"""Pins the oracle (oracle/quant_oracle.c) on the CPU.

- binary16 decode: all 65,536 encodings against the ldexp closed form, and
  round-to-nearest-even at every tie (backend/tests/test_kv_precision.c);
- block decode: Q4_K/Q6_K fixtures built from logical scales by an encoder
  independent of the decoder, exact (backend/tests/test_architectures.c:229-300),
  and power-of-two constant rows for Q4_0/Q8_0 (backend/tests/test_generation.c:79-103);
- scalar order: bit-exact against golden outputs of the reference's own
  nya_llm_matvec (tests/golden), and against the reference build itself when
  it is present;
- double oracle: against numpy brute force on small inputs.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from fyodor_amd import BF16, F16, F32, Q4_0, Q4_K, Q6_K, Q8_0, TYPE_NAMES, synth
from patterns import batch_inputs, constant_rows, k_quant_fixture, pass_input, pattern_matrix

GOLDEN = Path(__file__).resolve().parent / "golden"
ALL = [F32, F16, BF16, Q4_0, Q8_0, Q4_K, Q6_K]


def half_closed_form(h: int) -> float:
    e, f = (h >> 10) & 31, h & 1023
    v = np.ldexp(np.float64(1024 + f), e - 25) if e else np.ldexp(np.float64(f), -24)
    return -v if h & 0x8000 else v


def test_half_decode_exhaustive(oracle):
    for h in range(65536):
        got = oracle.half(h)
        if (h >> 10) & 31 == 31:
            assert np.isinf(got) if h & 1023 == 0 else np.isnan(got)
        else:
            assert got == half_closed_form(h) and np.signbit(got) == bool(h & 0x8000), h


def test_round_f16_ties_to_even(oracle):
    f32 = np.float32
    for h in range(0x7BFF):
        a, b = f32(half_closed_form(h)), f32(half_closed_form(h + 1))
        assert oracle.round_f16(float(a)) == a
        mid = f32((a + b) * f32(0.5))
        even = b if h & 1 else a
        for sign in (1, -1):
            s = f32(sign)
            assert oracle.round_f16(float(s * mid)) == s * even
            assert oracle.round_f16(float(s * np.nextafter(mid, f32(0)))) == s * a
            assert oracle.round_f16(float(s * np.nextafter(mid, f32(np.inf)))) == s * b
    assert np.isinf(oracle.round_f16(65520.0))
    assert oracle.round_f16(float(np.nextafter(f32(65520), f32(0)))) == 65504.0
    assert np.signbit(oracle.round_f16(-0.0)) and np.isnan(oracle.round_f16(float("nan")))


@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K"])
def test_k_quant_logical_fixture(oracle, kind):
    t = Q4_K if kind == "Q4_K" else Q6_K
    data, expected, x = k_quant_fixture(kind)
    assert np.array_equal(oracle.values(data, t, 1024), expected)
    y = oracle.matvec(data, t, x, 2, 512)
    exact = expected.reshape(2, 512).astype(np.float64) @ x.astype(np.float64)
    assert np.array_equal(y.astype(np.float64), exact)


@pytest.mark.parametrize("type_id", [Q4_0, Q8_0])
@pytest.mark.parametrize("value", [1.0, 0.03125, 0.015625])
def test_constant_rows(oracle, type_id, value):
    rows, cols = 3, 256
    w = constant_rows(type_id, rows, cols, value)
    assert np.all(oracle.values(w, type_id, rows * cols) == np.float32(value))
    x = (np.arange(cols) % 7 - 3).astype(np.float32) / np.float32(4)
    assert np.all(oracle.matvec(w, type_id, x, rows, cols) == np.float32(value * float(x.sum())))


def golden():
    arrays = np.load(GOLDEN / "reference_outputs.npz")
    manifest = json.loads((GOLDEN / "manifest.json").read_text())
    return arrays, manifest


@pytest.mark.parametrize("cols", [1024, 8192])
@pytest.mark.parametrize("type_id", ALL, ids=lambda t: TYPE_NAMES[t])
def test_scalar_order_matches_reference_golden(oracle, type_id, cols):
    arrays, manifest = golden()
    key = f"pattern_{TYPE_NAMES[type_id]}_{cols}"
    w = pattern_matrix(type_id, 65, cols)
    xs = [pass_input(cols, p) for p in range(3)]
    assert synth.digest(w, *xs) == manifest["pattern"][key], "input generator drifted"
    for p in range(3):
        y = oracle.matvec(w, type_id, xs[p], 65, cols)
        assert np.array_equal(y.view(np.uint32), arrays[key][p].view(np.uint32))


def test_batch_and_synthetic_golden(oracle):
    arrays, manifest = golden()
    for cols in (1024, 8192):
        w = pattern_matrix(Q4_K, 65, cols)
        y = oracle.matmul(w, Q4_K, batch_inputs(5, cols), 65, cols, 5)
        assert np.array_equal(y.view(np.uint32), arrays[f"batch_Q4_K_{cols}"].view(np.uint32))
    for case in manifest["synth"]:
        w = synth.weights(case["type"], case["rows"], case["cols"], case["seed"])
        x = synth.activations(case["batch"], case["cols"], case["seed"])
        assert synth.digest(w, x) == case["digest"], "synthetic generator drifted"
        y = oracle.matmul(w, case["type"], x, case["rows"], case["cols"], case["batch"], threads=4)
        assert np.array_equal(y.view(np.uint32), arrays[case["key"]].view(np.uint32)), case["key"]


@pytest.mark.parametrize("type_id", ALL, ids=lambda t: TYPE_NAMES[t])
def test_oracle_equals_reference_build(oracle, reference, type_id):
    for rows, cols, seed in [(17, 512, 1), (5, 4096, 2), (3, 768 if type_id not in (Q4_K, Q6_K) else 1024, 3)]:
        w = synth.weights(type_id, rows, cols, seed)
        x = synth.activations(1, cols, seed)[0]
        assert np.array_equal(oracle.matvec(w, type_id, x, rows, cols).view(np.uint32),
                              reference.matvec(w, type_id, x, rows, cols).view(np.uint32))
        idx = np.arange(0, rows * cols, 37)
        assert np.array_equal(oracle.values(w, type_id, rows * cols)[idx],
                              np.array([reference.value(w, type_id, int(i)) for i in idx], dtype=np.float32))


@pytest.mark.parametrize("type_id", ALL, ids=lambda t: TYPE_NAMES[t])
def test_double_oracle_brute_force(oracle, type_id):
    rows, cols = 3, 256
    w = synth.weights(type_id, rows, cols, 11)
    x = synth.activations(1, cols, 11)[0]
    vals = oracle.values(w, type_id, rows * cols).astype(np.float64).reshape(rows, cols)
    s, m = oracle.matvec_double(w, type_id, x, rows, cols)
    prods = vals * x.astype(np.float64)
    assert np.allclose(s, prods.sum(axis=1), rtol=0, atol=1e-12 * (1 + np.abs(prods).sum()))
    assert np.allclose(m, np.abs(prods).sum(axis=1), rtol=1e-15)


@pytest.mark.parametrize("type_id", ALL, ids=lambda t: TYPE_NAMES[t])
def test_dequant_equals_values(oracle, type_id):
    """orc_dequant (threaded, whole matrix) is element for element the pinned
    orc_value, for every thread split, and contract_sums equals the per-row
    double oracle."""
    rows, cols = 7, 512
    w = synth.weights(type_id, rows, cols, 21)
    vals = oracle.values(w, type_id, rows * cols).reshape(rows, cols)
    for threads in (1, 3, 16):
        got = oracle.dequant(w, type_id, rows, cols, threads=threads)
        assert np.array_equal(got.view(np.uint32), vals.view(np.uint32))
    x = synth.activations(3, cols, 22)
    s, m = oracle.contract_sums(w, type_id, x, rows, cols)
    for k in range(3):
        s1, m1 = oracle.matvec_double(w, type_id, x[k], rows, cols)
        assert np.allclose(s[k], s1, rtol=0, atol=1e-12 * (1 + m1.max()))
        assert np.allclose(m[k], m1, rtol=1e-13, atol=0)

"""Exact-result GPU fixtures from the reference's own tests, through the C ABI.

- K-quant blocks from logical scales: the GPU matvec equals the double dot
  exactly (backend/tests/test_architectures.c:281-298 requires this of the
  CUDA provider);
- Q4_0/Q8_0 constant rows with power-of-two scales (backend/tests/test_generation.c:79-103);
- every finite F16/BF16 encoding through a 65536 x 1 matvec
  (backend/tests/test_quant_kernels.c:27-49);
- y = (r+1)(b+1) for 65 rows x 8192 columns x 33 tokens over F32/F16/BF16/Q8_0,
  and BF16 transpose edges 33/65/257 x 5/31/33 (test_quant_kernels.c:55-136);
- F32 7x129 and 257x1025 with signed fractions within 1e-4 of double, batch
  33, and cached-weight reuse across alternating shapes (backend/tests/test_compute.c).
"""
import numpy as np
import pytest

from fyodor_amd import BF16, F16, F32, Q4_0, Q4_K, Q6_K, Q8_0, TYPE_NAMES
from patterns import constant_rows, k_quant_fixture

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K"])
def test_k_quant_fixture_exact(compute, kind):
    t = Q4_K if kind == "Q4_K" else Q6_K
    data, expected, x = k_quant_fixture(kind)
    y = compute.matvec_typed(data, 2, 512, t, x)
    exact = expected.reshape(2, 512).astype(np.float64) @ x.astype(np.float64)
    assert np.array_equal(y.astype(np.float64), exact)


@pytest.mark.parametrize("t", [Q4_0, Q8_0], ids=["Q4_0", "Q8_0"])
@pytest.mark.parametrize("value", [1.0, 0.03125, 0.015625])
def test_constant_rows_exact(compute, t, value):
    rows, cols = 7, 512
    w = constant_rows(t, rows, cols, value)
    x = (np.arange(cols) % 7 - 3).astype(np.float32) / np.float32(4)
    y = compute.matvec_typed(w, rows, cols, t, x)
    assert np.all(y == np.float32(value * float(x.sum())))


@pytest.mark.parametrize("t", [F16, BF16], ids=["F16", "BF16"])
def test_storage_edges_exhaustive(compute, oracle, t):
    mask = 0x7C00 if t == F16 else 0x7F80
    bits = np.arange(65536, dtype=np.uint32)
    bits = np.where((bits & mask) == mask, 0, bits).astype(np.uint16)
    data = bits.view(np.uint8).copy()
    y = compute.matvec_typed(data, 65536, 1, t, np.ones(1, dtype=np.float32))
    assert np.array_equal(y, oracle.values(data, t, 65536))


def encode_row_value(t, rows, cols, r):
    value = np.float32((r + 1) / 128)
    if t == F32:
        return np.full(cols, value, dtype=np.float32).view(np.uint8)
    bits = int(value.view(np.uint32))
    enc = bits >> 16 if t == BF16 else (((bits >> 23) - 112) << 10) | ((bits >> 13) & 1023)
    if t in (F16, BF16):
        return np.full(cols, enc, dtype=np.uint16).view(np.uint8)
    blk = np.array([0, 0x20] + [r + 1] * 32, dtype=np.uint8)   # d = 1/128
    return np.tile(blk, cols // 32)


@pytest.mark.parametrize("t", [F32, F16, BF16, Q8_0], ids=lambda t: TYPE_NAMES[t])
def test_chunked_matrix_exact(compute, t):
    rows, cols, batch = 65, 8192, 33
    w = np.concatenate([encode_row_value(t, rows, cols, r) for r in range(rows)])
    x = np.repeat((np.arange(1, batch + 1, dtype=np.float32) / np.float32(64))[:, None], cols, axis=1)
    out = np.full(rows * batch + 2, 12345, dtype=np.float32)
    y = compute.matmul_typed(w, rows, cols, t, x, batch, out=out[1:-1])
    assert out[0] == 12345 and out[-1] == 12345
    expected = np.outer(np.arange(1, batch + 1), np.arange(1, rows + 1)).astype(np.float32)
    assert np.array_equal(y, expected)


@pytest.mark.parametrize("cols,rows", [(33, 5), (65, 31), (257, 33)])
def test_bf16_transpose_edges(compute, cols, rows):
    batch = 33
    vals = (np.arange(1, rows + 1, dtype=np.float32) / np.float32(64))
    w = np.repeat((vals.view(np.uint32) >> 16).astype(np.uint16)[:, None], cols, axis=1).view(np.uint8).copy()
    x = np.repeat((np.arange(1, batch + 1, dtype=np.float32) / np.float32(64))[:, None], cols, axis=1)
    out = np.full(rows * batch + 2, 12345, dtype=np.float32)
    y = compute.matmul_typed(w, rows, cols, BF16, x, batch, out=out[1:-1])
    assert out[0] == 12345 and out[-1] == 12345
    expected = (cols * np.outer(np.arange(1, batch + 1), np.arange(1, rows + 1)) / 4096).astype(np.float32)
    assert np.array_equal(y, expected)


@pytest.mark.parametrize("rows,cols", [(7, 129), (257, 1025)])
def test_compute_f32_nonsquare(compute, rows, cols):
    w = ((np.arange(rows * cols) % 23) - 11).astype(np.float32) / np.float32(17)
    wd = w.reshape(rows, cols).astype(np.float64)
    for p in range(3):
        x = ((np.arange(cols) % 13) - 6 + p).astype(np.float32) / np.float32(7)
        y = compute.matvec_typed(w, rows, cols, F32, x)
        exp = wd @ x.astype(np.float64)
        assert np.all(np.abs(y - exp) <= 1e-4 * (1 + np.abs(exp)))
    i = np.arange(33 * cols)
    xb = ((((i * 3 + i // cols) % 13) - 6).astype(np.float32) / np.float32(7)).reshape(33, cols)
    y = compute.matmul_typed(w, rows, cols, F32, xb, 33)
    exp = xb.astype(np.float64) @ wd.T
    assert np.all(np.abs(y - exp) <= 1e-4 * (1 + np.abs(exp)))


def test_cached_weight_reuse_and_resizing(compute):
    small = np.arange(6, dtype=np.float32) / np.float32(10)
    large = ((np.arange(325) % 17) - 8).astype(np.float32) / np.float32(19)
    for p in range(6):
        rows, cols, w = (2, 3, small) if p % 2 == 0 else (5, 65, large)
        x = (np.arange(cols) + p).astype(np.float32) / np.float32(71)
        y = compute.matvec_typed(w, rows, cols, F32, x)
        exp = w.reshape(rows, cols).astype(np.float64) @ x.astype(np.float64)
        assert np.all(np.abs(y - exp) <= 1e-4 * (1 + np.abs(exp)))
    assert compute.name == "rocm"

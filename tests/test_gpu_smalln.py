"""The small-N MFMA path (batch 1..8) through the kernel library's C ABI.

- every batch 2..8 equals the same tokens of a batch of 8 bit for bit (the
  integer block dots are exact and the float epilogue does not depend on the
  batch), over partial 32-row tiles and short last Q8_0/Q4_0 column groups;
  where batch 1 runs on the same kernel the single tokens are equal too,
  where it runs on the batch-1 matvec (its own block order and 21-bit
  activation digits) they agree within 2e-6 of each row's magnitude;
- matrices wider than one launch's column chunk (20480 columns) against the
  double-precision oracle under the reference kernel contract's per-row bound;
- without a workspace the library runs a batch token by token, same result.
"""
import numpy as np
import pytest

from fyodor_amd import Q4_0, Q4_K, Q6_K, Q8_0, TYPE_NAMES, storage_bytes, synth
from checks import check_rows, rel_l2

pytestmark = pytest.mark.gpu

QUANT = [Q4_0, Q8_0, Q4_K, Q6_K]


@pytest.fixture(scope="module")
def hip():
    from fyodor_amd.hip import Kernels, Runtime
    rt = Runtime()
    return rt, Kernels(), rt.stream()


def run(hip, w, t, rows, cols, x, batch, workspace=True):
    rt, kern, stream = hip
    need = kern.workspace_bytes(t, rows, cols, batch) if workspace else 0
    wdev, xdev = rt.malloc(storage_bytes(t, rows, cols)), rt.malloc(x.nbytes)
    ydev, work = rt.malloc(4 * rows * batch), rt.malloc(max(need, 16))
    try:
        rt.upload(wdev, kern.device_weights(w, t, rows, cols))
        rt.upload(xdev, np.ascontiguousarray(x, dtype=np.float32))
        kern.matmul(wdev, t, rows, cols, xdev, ydev, batch, work if need else 0, need, stream)
        rt.sync(stream)
        return rt.download(ydev, np.empty((batch, rows), dtype=np.float32))
    finally:
        for p in (wdev, xdev, ydev, work):
            rt.free(p)


@pytest.mark.parametrize("t", QUANT, ids=lambda t: TYPE_NAMES[t])
def test_batches_equal_single_tokens(hip, t):
    rows = 200
    cols = 800 if t in (Q4_0, Q8_0) else 1024
    w = synth.weights(t, rows, cols, 300 + t)
    x = synth.activations(8, cols, 301 + t)
    single = np.stack([run(hip, w, t, rows, cols, x[k:k + 1], 1)[0] for k in range(8)])
    full = run(hip, w, t, rows, cols, x, 8)
    for batch in range(2, 8):
        y = run(hip, w, t, rows, cols, x[:batch], batch)
        assert np.array_equal(y, full[:batch]), f"batch {batch}"
    if hip[1].kernel_name(t, rows, cols, 1) == "smalln_mfma":
        assert np.array_equal(full, single)
    else:
        scale = np.abs(single).max(axis=1, keepdims=True) + 1e-30
        assert np.all(np.abs(full - single) <= 2e-6 * scale)
    assert np.array_equal(run(hip, w, t, rows, cols, x[:5], 5, workspace=False), single[:5])


@pytest.mark.parametrize("t", QUANT, ids=lambda t: TYPE_NAMES[t])
@pytest.mark.parametrize("batch", [1, 3, 8])
def test_wide_rows_span_launches(hip, oracle, t, batch):
    rows, cols = 40, 20480
    w = synth.weights(t, rows, cols, 400 + t)
    x = synth.activations(batch, cols, 401 + t)
    y = run(hip, w, t, rows, cols, x, batch)
    for k in range(batch):
        check_rows(oracle, w, t, x[k], rows, cols, y[k])
        assert rel_l2(y[k], oracle.matvec(w, t, x[k], rows, cols)) <= 1e-5

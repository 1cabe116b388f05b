"""The small-N MFMA path (batch 1..8) through the kernel library's C ABI.

- every batch 2..8 equals the same tokens of a batch of 8 bit for bit (the
  integer block dots are exact and the float epilogue does not depend on the
  batch), over partial 32-row tiles and short last Q8_0/Q4_0 column groups;
  where batch 1 runs on the same kernel the single tokens are equal too,
  where it runs on the batch-1 matvec (its own block order and 21-bit
  activation digits) they agree within 2e-6 of each row's magnitude;
- matrices wider than one launch's column chunk (20480 columns) against the
  double-precision oracle under the reference kernel contract's per-row bound;
- without a workspace the library runs a batch token by token, same result
  (or, where the row-balanced kernel takes the shape, the batch itself: it
  needs no workspace).
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
    # Without a workspace: the row-balanced kernel needs none; otherwise the
    # tokens run one at a time.
    y5 = run(hip, w, t, rows, cols, x[:5], 5, workspace=False)
    assert np.array_equal(y5, full[:5] if hip[1].kernel_name(t, rows, cols, 5) == "smalln_rows" else single[:5])


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


ROWS_TYPES = [Q4_0, Q8_0, Q4_K]


@pytest.mark.parametrize("t", ROWS_TYPES, ids=lambda t: TYPE_NAMES[t])
@pytest.mark.parametrize("rows,cols", [(200, 4096), (9000, 1024), (40, 256), (16384, 512), (72, 11008),
                                       (20000, 256)],
                         ids=["partial-tile", "two-virtual-tiles-ragged", "one-group", "two-virtual-tiles",
                              "groups-per-wave", "tile-per-workgroup"])
def test_rows_kernel_against_oracle(hip, oracle, t, rows, cols):
    """The row-balanced small-N kernel (activation digits made in the kernel,
    one exponent per token and 256-column group) under the reference
    contract's per-row bound, tokens spanning 2^-40 .. 2^44 in magnitude and
    single groups 2^-20 below the rest of their token."""
    assert hip[1].kernel_name(t, rows, cols, 8) == "smalln_rows"
    w = synth.weights(t, rows, cols, 500 + t)
    x = synth.activations(8, cols, 501 + t)
    x *= np.float32(2.0) ** np.arange(-40, 56, 12, dtype=np.float32)[:, None]
    x[3, 256:512] *= np.float32(2.0 ** -20)
    y = run(hip, w, t, rows, cols, x, 8)
    for k in range(8):
        check_rows(oracle, w, t, x[k], rows, cols, y[k])
        assert rel_l2(y[k], oracle.matvec(w, t, x[k], rows, cols)) <= 1e-5
    assert np.array_equal(run(hip, w, t, rows, cols, x[:3], 3), y[:3])


@pytest.mark.parametrize("rows,cols", [(200, 4096), (40, 256), (72, 11008), (9000, 512)],
                         ids=["partial-tile", "one-group", "groups-per-wave", "tile-per-workgroup"])
def test_rows_kernel_q6k_against_oracle(hip, oracle, rows, cols):
    """Q6_K on the row kernel (each lane half with its own 16-column
    scales; rows wider than 4096 columns at eight slots on eight wavefronts)
    under the contract bound, tokens spanning 2^-40 .. 2^44."""
    t = Q6_K
    assert hip[1].kernel_name(t, rows, cols, 8) == "smalln_rows"
    w = synth.weights(t, rows, cols, 700)
    x = synth.activations(8, cols, 701)
    x *= np.float32(2.0) ** np.arange(-40, 56, 12, dtype=np.float32)[:, None]
    for batch in (8, 3):
        y = run(hip, w, t, rows, cols, x[:batch], batch)
        for k in range(batch):
            check_rows(oracle, w, t, x[k], rows, cols, y[k])
            assert rel_l2(y[k], oracle.matvec(w, t, x[k], rows, cols)) <= 1e-5


@pytest.mark.parametrize("t", ROWS_TYPES + [Q6_K], ids=lambda t: TYPE_NAMES[t])
def test_nonfinite_token(hip, t):
    """An inf or NaN in one token's x makes every output of that token
    non-finite and leaves the other tokens as they were."""
    rows, cols = 256, 1024
    w = synth.weights(t, rows, cols, 600 + t)
    x = synth.activations(4, cols, 601 + t)
    clean = run(hip, w, t, rows, cols, x, 4)
    x[1, 300] = np.inf
    x[2, 5] = np.nan
    y = run(hip, w, t, rows, cols, x, 4)
    assert not np.isfinite(y[1]).any() and not np.isfinite(y[2]).any()
    assert np.array_equal(y[[0, 3]], clean[[0, 3]])
    for k in (1, 2):
        assert not np.isfinite(run(hip, w, t, rows, cols, x[k:k + 1], 1)).any()

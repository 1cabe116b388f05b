"""The prefill GEMM (batches above 8): fp16 MFMA for Q4_0 / Q8_0 / Q4_K,
int8 MFMA for Q6_K.

- prefill shapes of the 8B-class projections at batch 128..512: sampled
  tokens (both tile edges included) against the double-precision oracle
  under the reference kernel contract's per-row bound and at relative
  L2 <= 1e-5 against the scalar oracle;
- batch and row tails (batch 9, 127..129, 257; 200 rows = one full and one
  partial weight tile) with canaries on both sides of the output;
- through the kernel library's C ABI: the GEMM (workspace given) against the
  same request run through the small-N path (int8 activation digits; both
  represent x to about 2^-22 and differ in fp32 summation order), and the
  workspace size it asks for.
"""
import numpy as np
import pytest

from fyodor_amd import Q4_0, Q4_K, Q6_K, Q8_0, TYPE_NAMES, storage_bytes, synth
from checks import check_rows, rel_l2
from patterns import batch_inputs, pattern_matrix

pytestmark = pytest.mark.gpu

QUANT = [Q4_0, Q8_0, Q4_K, Q6_K]

PREFILL = [
    (Q4_K, 14336, 4096, 512),
    (Q4_K, 4096, 14336, 128),
    (Q8_0, 4096, 4096, 512),
    (Q6_K, 4096, 14336, 128),
    (Q4_0, 11008, 4096, 256),
]


@pytest.mark.parametrize("type_id,rows,cols,batch", PREFILL,
                         ids=[f"{TYPE_NAMES[t]}-{r}x{c}-n{b}" for t, r, c, b in PREFILL])
def test_prefill_shapes(compute, oracle, type_id, rows, cols, batch):
    seed = type_id * 7919 + rows + 3 * cols + batch
    w = synth.weights(type_id, rows, cols, seed)
    x = synth.activations(batch, cols, seed)
    y = compute.matmul_typed(w, rows, cols, type_id, x, batch)
    assert np.all(np.isfinite(y))
    for token in sorted({0, 1, 31, 32, 127, batch // 2, batch - 1}):
        check_rows(oracle, w, type_id, x[token], rows, cols, y[token])
        expected = oracle.matvec(w, type_id, x[token], rows, cols)
        assert rel_l2(y[token], expected) <= 1e-5, f"token {token}"


@pytest.mark.parametrize("type_id", QUANT, ids=lambda t: TYPE_NAMES[t])
@pytest.mark.parametrize("batch", [9, 127, 128, 129, 257])
def test_batch_and_row_tails(compute, oracle, type_id, batch):
    rows, cols = 200, 512
    w = pattern_matrix(type_id, rows, cols)
    x = batch_inputs(batch, cols) * np.float32(1.5) - np.float32(0.25)
    out = np.full(batch * rows + 2, 12345, dtype=np.float32)
    compute.matmul_typed(w, rows, cols, type_id, x, batch, out=out[1:-1])
    assert out[0] == 12345 and out[-1] == 12345
    y = out[1:-1].reshape(batch, rows)
    for token in sorted({0, batch // 3, batch - 2, batch - 1}):
        check_rows(oracle, w, type_id, x[token], rows, cols, y[token])


@pytest.fixture(scope="module")
def hip():
    from fyodor_amd.hip import Kernels, Runtime
    rt = Runtime()
    return rt, Kernels(), rt.stream()


@pytest.mark.parametrize("type_id", QUANT, ids=lambda t: TYPE_NAMES[t])
def test_prefill_matches_tiled_path(hip, type_id):
    rt, kern, stream = hip
    rows, cols, batch = 384, 2048, 40
    w = synth.weights(type_id, rows, cols, 77 + type_id)
    x = synth.activations(batch, cols, 78 + type_id)
    need = kern.workspace_bytes(type_id, rows, cols, batch)
    if type_id == Q6_K:
        assert need == cols // 32 * 136 * 64      # digits, batch rounded up to 32 tokens
        assert kern.kernel_name(type_id, rows, cols, batch) == "prefill_mfma"
    else:
        assert need == 64 * (4 * cols + cols // 32 * 4 + 4)   # fp16 pieces of 64 tokens
        assert kern.kernel_name(type_id, rows, cols, batch) == "prefill_f16"
    wdev, xdev = rt.malloc(storage_bytes(type_id, rows, cols)), rt.malloc(x.nbytes)
    ydev, work = rt.malloc(4 * rows * batch), rt.malloc(need)
    try:
        rt.upload(wdev, kern.device_weights(w, type_id, rows, cols))
        rt.upload(xdev, x)
        kern.matmul(wdev, type_id, rows, cols, xdev, ydev, batch, work, need, stream)
        rt.sync(stream)
        pre = rt.download(ydev, np.empty((batch, rows), dtype=np.float32))
        kern.matmul(wdev, type_id, rows, cols, xdev, ydev, batch, 0, 0, stream)
        rt.sync(stream)
        tiled = rt.download(ydev, np.empty((batch, rows), dtype=np.float32))
        # A workspace one byte short is refused by the prefill GEMM: tiled again.
        kern.matmul(wdev, type_id, rows, cols, xdev, ydev, batch, work, need - 1, stream)
        rt.sync(stream)
        short = rt.download(ydev, np.empty((batch, rows), dtype=np.float32))
    finally:
        for p in (wdev, xdev, ydev, work):
            rt.free(p)
    # Without the GEMM's workspace the batch runs 8 tokens at a time: on the
    # row-balanced small-N kernel where it takes the shape (no workspace
    # either way); else without a workspace token by token, on the batch-1
    # matvec where the type has one (its own rounding) or on the same small-N
    # kernel as the batches of 8 the short workspace gets.
    if kern.kernel_name(type_id, rows, cols, 8) == "smalln_rows" or kern.kernel_name(type_id, rows, cols, 1) == "smalln_mfma":
        assert np.array_equal(short, tiled)
    else:
        assert rel_l2(short, tiled) <= 2e-6
    assert rel_l2(pre, tiled) <= 2e-6

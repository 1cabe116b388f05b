"""Dense F32 / F16 / BF16 batches above 8 on the fp32-MFMA GEMM
(nya_hip_matmul, kernel "dense_gemm"), through the kernel library's C ABI:

- under the reference kernel contract (backend/tests/test_quant_kernels.c:13-25,
  :138-213): every token and row within 1e-6 (1 + sum |w x|) of the double
  sum of the decoded products, and within relative L2 1e-5 of the scalar
  oracle (the reference's F32 path accumulates in double,
  backend/core/llm_quant.c:161-204), at batches 9 .. 512, rows that are not
  a multiple of the 128-row tile, tokens that are not a multiple of 64, and
  column counts with a short last 32-column chunk or rows that are not
  16-byte aligned (the element-by-element loads);
- an exact fixture: small integer weights and activations, whose products
  and sums are exact in fp32, give the exact integer result;
- canaries on both sides of the output stay untouched;
each with the workspace nya_hip_workspace_bytes asks for (small tile counts
split the columns over several workgroups, added in order by a second
launch) and without one (a workgroup per tile over all columns).
"""
import numpy as np
import pytest

from fyodor_amd import BF16, F16, F32, TYPE_NAMES, storage_bytes, synth
from fyodor_amd.hip import Kernels, Runtime
from oracle import host_threads

pytestmark = pytest.mark.gpu

SHAPES = [(300, 1024, 9), (129, 1000, 40), (1000, 8192, 65), (64, 33, 17), (100, 1002, 12), (4096, 4096, 512),
          (257, 4104, 100)]


@pytest.fixture(scope="module")
def hip():
    rt = Runtime()
    return rt, Kernels(), rt.stream()


def run(hip, w, t, x, rows, cols, batch, workspace=True):
    """nya_hip_matmul on device copies; the output with one canary float on
    each side. With the workspace it asks for, small tile counts split the
    columns over several workgroups; without, one workgroup per tile."""
    rt, kern, stream = hip
    assert kern.kernel_name(t, rows, cols, batch) == "dense_gemm"
    need = kern.workspace_bytes(t, rows, cols, batch) if workspace else 0
    wd, xd = rt.malloc(max(w.nbytes, 16)), rt.malloc(x.nbytes)
    out, ws = rt.malloc(4 * (batch * rows + 2)), rt.malloc(max(need, 16))
    try:
        rt.upload(wd, w)
        rt.upload(xd, np.ascontiguousarray(x, dtype=np.float32))
        rt.upload(out, np.full(batch * rows + 2, 12345.0, dtype=np.float32))
        kern.matmul(wd, t, rows, cols, xd, out + 4, batch, ws if need else 0, need, stream)
        rt.sync(stream)
        y = rt.download(out, np.empty(batch * rows + 2, dtype=np.float32))
    finally:
        for p in (wd, xd, out, ws):
            rt.free(p)
    assert y[0] == 12345.0 and y[-1] == 12345.0, "canary overwritten"
    return y[1:-1].reshape(batch, rows)


@pytest.mark.parametrize("t", [F32, F16, BF16], ids=lambda t: TYPE_NAMES[t])
@pytest.mark.parametrize("rows,cols,batch", SHAPES, ids=[f"{r}x{c}-m{b}" for r, c, b in SHAPES])
def test_dense_gemm_contract(hip, oracle, t, rows, cols, batch):
    seed = 41 * t + rows + cols + batch
    w = synth.weights(t, rows, cols, seed)
    x = synth.activations(batch, cols, seed + 1)
    s, m = oracle.contract_sums(w, t, x, rows, cols)
    scalar = oracle.matmul(w, t, x, rows, cols, batch, threads=host_threads())
    for workspace in (True, False):
        print(f"dense_gemm {TYPE_NAMES[t]} {rows}x{cols} batch {batch} workspace {workspace}", flush=True)
        y = run(hip, w, t, x, rows, cols, batch, workspace)
        assert np.all(np.isfinite(y))
        err = np.abs(y.astype(np.float64) - s)
        bad = err > 1e-6 * (1 + m)
        assert not bad.any(), f"{int(bad.sum())} outputs outside the contract bound, first at {np.argwhere(bad)[0]}"
        num = np.linalg.norm(y.astype(np.float64) - scalar, axis=1)
        den = np.linalg.norm(scalar.astype(np.float64), axis=1)
        assert np.all(num <= 1e-5 * den), f"relative L2 {float((num / den).max()):.3g}"


@pytest.mark.parametrize("t", [F32, F16, BF16], ids=lambda t: TYPE_NAMES[t])
def test_dense_gemm_exact_integers(hip, t):
    """Weights in -8..7 and activations in -16..15: every product and every
    partial sum is an integer below 2^24, so fp32 accumulation is exact."""
    rows, cols, batch = 200, 2048, 70
    rng = np.random.default_rng(7 + t)
    wv = rng.integers(-8, 8, size=(rows, cols)).astype(np.float32)
    x = rng.integers(-16, 16, size=(batch, cols)).astype(np.float32)
    if t == F32:
        w = wv.view(np.uint8).reshape(-1).copy()
    elif t == F16:
        w = wv.astype(np.float16).view(np.uint8).reshape(-1).copy()
    else:
        w = (wv.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(-1).copy()
    assert w.nbytes == storage_bytes(t, rows, cols)
    exact = x.astype(np.float64) @ wv.astype(np.float64).T
    for workspace in (True, False):
        y = run(hip, w, t, x, rows, cols, batch, workspace)
        assert np.array_equal(y.astype(np.float64), exact)

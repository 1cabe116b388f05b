"""nya_hip_matmul_static, the entry point that allocates nothing (its
kernels' scratch is the library's static device array), against
nya_hip_matmul with a workspace of the size it asks for, through the kernel
library's C ABI. Each case makes two calls in a row, the second with a
smaller input, so the second reads a scratch array the first left full;
the outputs must equal the workspace entry point's bit for bit (same
kernels on the same tokens). Cases: the fp16 prefill GEMM in one chunk and
in two (4096 x 14336 at 2048 tokens needs 121 MB of scratch against the
array's 64 MiB), the int8 Q6_K prefill, the small-N tile kernel's digits
(the only batch of 2..8 that uses scratch) and the batch-1 matvec; and
rows too wide for any GEMM chunk to fit the array.
"""
import numpy as np
import pytest

from fyodor_amd import Q4_K, Q6_K, Q8_0, TYPE_NAMES, storage_bytes, synth
from fyodor_amd.hip import Kernels, Runtime

pytestmark = pytest.mark.gpu

SCRATCH = 64 << 20

CASES = [
    (Q4_K, 14336, 4096, (2048, 40)),
    (Q4_K, 4096, 14336, (2048, 100)),
    (Q6_K, 4096, 4096, (300, 20)),
    (Q4_K, 14336, 8192, (8, 3)),
    (Q8_0, 4096, 4096, (1, 1)),
]


@pytest.fixture(scope="module")
def hip():
    rt = Runtime()
    return rt, Kernels(), rt.stream()


@pytest.mark.parametrize("t,rows,cols,batches", CASES,
                         ids=[f"{TYPE_NAMES[t]}-{r}x{c}-m{b[0]}-then-{b[1]}" for t, r, c, b in CASES])
def test_static_matches_workspace_entry(hip, t, rows, cols, batches):
    rt, kern, stream = hip
    w = synth.weights(t, rows, cols, 300 + t + rows)
    wd = rt.malloc(storage_bytes(t, rows, cols))
    rt.upload(wd, kern.device_weights(w, t, rows, cols))
    try:
        for call, batch in enumerate(batches):
            x = synth.activations(batch, cols, 301 + call)
            need = kern.workspace_bytes(t, rows, cols, batch)
            if call == 0 and (t, rows, cols) == (Q4_K, 4096, 14336):
                assert need > SCRATCH, "this case must run in more than one chunk"
            xd, yd, ws = rt.malloc(x.nbytes), rt.malloc(4 * rows * batch), rt.malloc(max(need, 16))
            try:
                rt.upload(xd, x)
                kern.matmul(wd, t, rows, cols, xd, yd, batch, ws, need, stream)
                rt.sync(stream)
                expected = rt.download(yd, np.empty((batch, rows), dtype=np.float32))
                rt.upload(yd, np.full((batch, rows), np.nan, dtype=np.float32))
                kern.matmul_static(wd, t, rows, cols, xd, yd, batch, stream)
                rt.sync(stream)
                got = rt.download(yd, np.empty((batch, rows), dtype=np.float32))
            finally:
                for p in (xd, yd, ws):
                    rt.free(p)
            assert np.all(np.isfinite(got)), f"call {call}: outputs left unwritten"
            assert np.array_equal(got.view(np.uint32), expected.view(np.uint32)), f"call {call} (batch {batch})"
    finally:
        rt.free(wd)


def test_static_rows_too_wide_for_a_gemm_chunk(hip):
    """Q4_K 8192 x 262144: 64 tokens of the GEMM's workspace need about 69 MB,
    more than the array, so the static entry runs batch 24 (then 9) as
    8-token launches; nya_hip_matmul without a workspace takes the same
    launches, so the outputs are equal bit for bit."""
    rt, kern, stream = hip
    t, rows, cols = Q4_K, 8192, 262144
    assert kern.workspace_bytes(t, rows, cols, 64) > SCRATCH
    w = synth.weights(t, rows, cols, 311)
    wd = rt.malloc(storage_bytes(t, rows, cols))
    rt.upload(wd, kern.device_weights(w, t, rows, cols))
    del w
    try:
        for call, batch in enumerate((24, 9)):
            x = synth.activations(batch, cols, 312 + call)
            xd, yd = rt.malloc(x.nbytes), rt.malloc(4 * rows * batch)
            try:
                rt.upload(xd, x)
                kern.matmul(wd, t, rows, cols, xd, yd, batch, 0, 0, stream)
                rt.sync(stream)
                expected = rt.download(yd, np.empty((batch, rows), dtype=np.float32))
                rt.upload(yd, np.full((batch, rows), np.nan, dtype=np.float32))
                kern.matmul_static(wd, t, rows, cols, xd, yd, batch, stream)
                rt.sync(stream)
                got = rt.download(yd, np.empty((batch, rows), dtype=np.float32))
            finally:
                rt.free(xd)
                rt.free(yd)
            assert np.all(np.isfinite(got)), f"call {call}: outputs left unwritten"
            assert np.array_equal(got.view(np.uint32), expected.view(np.uint32)), f"call {call} (batch {batch})"
    finally:
        rt.free(wd)


def test_static_declines_like_the_workspace_entry(hip):
    """Declined shapes are declined before anything is enqueued (status 1)."""
    rt, kern, stream = hip
    L = kern.lib
    assert L.nya_hip_matmul_static(0, Q8_0, 3, 32, 16, 16, 1, stream) == 1
    assert L.nya_hip_matmul_static(1 << 20, Q4_K, 3, 100, 1 << 20, 1 << 20, 1, stream) == 1

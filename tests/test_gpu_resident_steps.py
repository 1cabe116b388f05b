"""The resident decoder steps of libfyodor_hip.so (include/fyodor_hip.h),
each called through the C-ABI on an MI355X and compared with a float64
numpy statement of the engine's step (backend/core/llm_cpu.c:71-104,
:298-341, :429-436, :491-511) on seeded inputs:

- dequant_row: bit-exact against the oracle's GGUF decoder, every type;
- rms_norm (with and without the residual add, on the vector and scalar
  paths): within 2e-6 (1 + |ref|);
- rope_qkv (q rotated in place, k rotated into the key slot, v copied):
  within 2e-6 (1 + |ref|), the v copy exact;
- attention at head widths 64 / 80 / 128 / 256, grouped and ungrouped heads,
  lengths from 1 through the LDS limit (8192) into the global-scratch path:
  within 1e-5 (1 + |ref|);
- silu_mul: within 2e-6 (1 + |ref|).
The bounds are fp32 rounding over these sums, far inside the engine's own
inference bounds (logits 5e-4 (1 + |ref|))."""
import ctypes

import numpy as np
import pytest

from fyodor_amd import BF16, F16, F32, Q4_0, Q4_K, Q6_K, Q8_0, storage_bytes, synth
from fyodor_amd.hip import Kernels, Runtime

pytestmark = pytest.mark.gpu

_up, _sz = ctypes.c_uint64, ctypes.c_size_t


@pytest.fixture(scope="module")
def env():
    rt, kern = Runtime(), Kernels()
    L = kern.lib
    L.nya_hip_dequant_row.argtypes = [_up, ctypes.c_uint, _sz, _sz, _sz, _up, _up]
    L.nya_hip_rms_norm.argtypes = [_up, _up, _up, _up, _sz, ctypes.c_float, _up]
    L.nya_hip_rope_qkv.argtypes = [_up, _sz, _sz, _sz, _up, _sz, _up, _up, _up]
    L.nya_hip_attention.argtypes = [_up, _up, _up, _up, _up, _sz, _sz, _sz, _sz, ctypes.c_float, _up]
    L.nya_hip_silu_mul.argtypes = [_up, _up, _sz, _up]
    stream = rt.stream()
    yield rt, L, stream
    rt.sync(stream)


class Dev:
    """Device copies of host arrays, freed together."""

    def __init__(self, rt):
        self.rt, self.ptrs = rt, []

    def put(self, a: np.ndarray, extra: int = 0) -> int:
        p = self.rt.malloc(a.nbytes + extra + 16)
        self.ptrs.append(p)
        self.rt.upload(p + extra, np.ascontiguousarray(a))
        return p + extra

    def empty(self, nbytes: int) -> int:
        p = self.rt.malloc(nbytes + 16)
        self.ptrs.append(p)
        return p

    def get(self, p: int, like: np.ndarray) -> np.ndarray:
        return self.rt.download(p, np.empty_like(like))

    def close(self):
        for p in self.ptrs:
            self.rt.free(p)


def scaled_error(got, ref):
    return float(np.max(np.abs(got.astype(np.float64) - ref) / (1 + np.abs(ref))))


@pytest.mark.parametrize("type_id", [F32, F16, BF16, Q8_0, Q4_0, Q4_K, Q6_K])
def test_dequant_row_exact(env, oracle, type_id):
    rt, L, stream = env
    rows, cols = 7, 512
    w = synth.weights(type_id, rows, cols, seed=40 + type_id)
    ref = oracle.dequant(w, type_id, rows, cols).reshape(rows, cols)
    dev = Dev(rt)
    try:
        wd, out = dev.put(w), dev.empty(4 * cols)
        for row in (0, 3, rows - 1):
            assert L.nya_hip_dequant_row(wd, type_id, rows, cols, row, out, stream) == 0
            rt.sync(stream)
            got = dev.get(out, np.empty(cols, np.float32))
            assert np.array_equal(got.view(np.uint32), ref[row].view(np.uint32)), f"row {row}"
        assert L.nya_hip_dequant_row(wd, type_id, rows, cols, rows, out, stream) == 1   # row out of range
    finally:
        dev.close()


@pytest.mark.parametrize("n,offset", [(4096, 0), (4098, 0), (4096, 4)], ids=["vector", "ragged", "misaligned"])
@pytest.mark.parametrize("residual", [False, True])
def test_rms_norm(env, n, offset, residual):
    rt, L, stream = env
    rng = np.random.default_rng(n + offset)
    x, r = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    eps = 1e-5
    xs32 = (x + r if residual else x).astype(np.float32)
    xs = xs32.astype(np.float64)
    scale = 1.0 / np.sqrt(np.sum(xs * xs) / n + eps)
    ref = xs32.astype(np.float64) * np.float32(scale) * w
    dev = Dev(rt)
    try:
        xd, rd, wd, od = dev.put(x, offset), dev.put(r, offset), dev.put(w), dev.empty(4 * n)
        assert L.nya_hip_rms_norm(xd, rd if residual else 0, wd, od, n, eps, stream) == 0
        rt.sync(stream)
        assert scaled_error(dev.get(od, x), ref) <= 2e-6
        assert np.array_equal(dev.get(xd, x), xs32)      # the residual add written back (or x untouched)
    finally:
        dev.close()


@pytest.mark.parametrize("heads,kv_heads,width", [(32, 8, 128), (4, 4, 64), (6, 2, 80)])
def test_rope_qkv(env, heads, kv_heads, width):
    rt, L, stream = env
    rng = np.random.default_rng(heads * width)
    qkv = rng.standard_normal((heads + 2 * kv_heads) * width).astype(np.float32)
    pairs = width // 2
    freq = (10000.0 ** (-np.arange(pairs) / pairs)).astype(np.float32)
    position = 1234
    angle = (np.float32(position) * freq).astype(np.float64)
    c, s = np.cos(angle), np.sin(angle)

    def rotate(v):
        v = v.reshape(-1, pairs, 2).astype(np.float64)
        a, b = v[..., 0], v[..., 1]
        return np.stack([a * c - b * s, a * s + b * c], -1).reshape(-1)

    q, k, v = np.split(qkv, [heads * width, (heads + kv_heads) * width])
    dev = Dev(rt)
    try:
        qd, fd = dev.put(qkv), dev.put(freq)
        kd, vd = dev.empty(k.nbytes), dev.empty(v.nbytes)
        assert L.nya_hip_rope_qkv(qd, heads, kv_heads, width, fd, position, kd, vd, stream) == 0
        rt.sync(stream)
        out = dev.get(qd, qkv)
        assert scaled_error(out[:q.size], rotate(q)) <= 2e-6
        assert np.array_equal(out[q.size:], qkv[q.size:])                 # k and v left in place
        assert scaled_error(dev.get(kd, k), rotate(k)) <= 2e-6
        assert np.array_equal(dev.get(vd, v), v)
    finally:
        dev.close()


def attention_ref(q, keys, values, heads, kv_heads, width, length, scale):
    q = q.reshape(heads, width).astype(np.float64)
    k = keys[:length].reshape(length, kv_heads, width).astype(np.float64)
    v = values[:length].reshape(length, kv_heads, width).astype(np.float64)
    group = heads // kv_heads
    out = np.empty((heads, width))
    for h in range(heads):
        s = k[:, h // group, :] @ q[h] * scale
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ v[:, h // group, :]
    return out.reshape(-1)


@pytest.mark.parametrize("heads,kv_heads,width,length", [
    (32, 8, 128, 1), (32, 8, 128, 37), (32, 8, 128, 1000), (8, 8, 64, 300), (6, 2, 80, 129), (4, 1, 256, 513),
    (8, 2, 128, 8192), (8, 2, 128, 9000),
])
def test_attention(env, heads, kv_heads, width, length):
    rt, L, stream = env
    rng = np.random.default_rng(length * 7 + width)
    capacity = length + 5
    q = rng.standard_normal(heads * width).astype(np.float32)
    keys = rng.standard_normal((capacity, kv_heads * width)).astype(np.float32)
    values = rng.standard_normal((capacity, kv_heads * width)).astype(np.float32)
    scale = float(1 / np.sqrt(np.float32(width)))
    ref = attention_ref(q, keys, values, heads, kv_heads, width, length, np.float32(scale))
    dev = Dev(rt)
    try:
        qd, kd, vd = dev.put(q), dev.put(keys), dev.put(values)
        od, sd = dev.empty(q.nbytes), dev.empty(4 * heads * length)
        assert L.nya_hip_attention(qd, kd, vd, od, sd, heads, kv_heads, width, length, scale, stream) == 0
        rt.sync(stream)
        err = scaled_error(dev.get(od, q), ref)
        print(f"attention {heads}/{kv_heads} x {width}, length {length}: scaled error {err:.3g}", flush=True)
        assert err <= 1e-5
    finally:
        dev.close()


def test_attention_declines_wide_heads(env):
    rt, L, stream = env
    dev = Dev(rt)
    try:
        p = dev.empty(4 * 4 * 512)
        assert L.nya_hip_attention(p, p, p, p, p, 2, 2, 512, 1, 1.0, stream) == 1
    finally:
        dev.close()


def test_silu_mul(env):
    rt, L, stream = env
    rng = np.random.default_rng(5)
    n = 14336
    g, u = (4 * rng.standard_normal(n)).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    dev = Dev(rt)
    try:
        gd, ud = dev.put(g), dev.put(u)
        assert L.nya_hip_silu_mul(gd, ud, n, stream) == 0
        rt.sync(stream)
        assert scaled_error(dev.get(gd, g), ref) <= 2e-6
    finally:
        dev.close()

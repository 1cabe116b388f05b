"""The resident decoder steps of libfyodor_hip.so (include/fyodor_hip.h),
each called through the C-ABI on an MI355X over one and several tokens, and
compared with a float64 numpy statement of the engine's step
(backend/core/llm_cpu.c:71-104, :298-341, :429-436, :491-511) on seeded
inputs:

- step: the decode slot holds the token id and position;
- embed: bit-exact against the oracle's GGUF decoder, every type; an id past
  the matrix gives a zero row;
- rms_norm (with and without the residual add, vector and scalar paths,
  several rows): within 2e-6 (1 + |ref|);
- rope_qkv (fused q|k|v rows and separate q / k,v blocks; q rotated in place,
  k rotated into its cache slot, v copied; a position past the cache leaves
  everything alone): within 2e-6 (1 + |ref|), the v copy exact;
- attention at head widths 64 / 80 / 128 / 256, grouped and ungrouped heads,
  one query and causal runs of several, lengths from 1 through the LDS limit
  (8192) into the global-scratch path: within 1e-5 (1 + |ref|);
- silu_mul (fused [gate | up] rows, separate blocks, in place for one
  token): within 2e-6 (1 + |ref|);
- matvec_normed (the residual add and RMS norm folded into a one-token
  product): y and the updated residual bit for bit those of rms_norm
  followed by nya_hip_matmul, with and without the residual add, for the
  quantized types at q|k|v shapes; declined (1) past 32 rows per CU or 4096
  columns;
- matvec_normed_rope (the same with rope_qkv in its epilogue): y and the
  whole key / value cache bit for bit matvec_normed followed by rope_qkv,
  for a position inside the cache and one past it;
- matvec_swiglu (a one-token gate|up product over 16-row-interleaved gate and
  up rows with silu(g) * u as output) bit for bit nya_hip_matmul followed by
  silu_pairs, and silu_pairs within 2e-6 (1 + |ref|) of float64;
- matvec_gated (the gated SiLU folded into a one-token down product): bit
  for bit the output of silu_mul followed by nya_hip_matmul, for every
  quantized type at down-projection shapes (wide rows, chunked rows, a
  ragged last tile), and declined (1) where the row kernel does not run.
The bounds are fp32 rounding over these sums, far inside the engine's own
inference bounds (logits 5e-4 (1 + |ref|))."""
import ctypes

import numpy as np
import pytest

from fyodor_amd import BF16, F16, F32, Q4_0, Q4_K, Q6_K, Q8_0, TYPE_NAMES, synth
from fyodor_amd.hip import Kernels, Runtime

pytestmark = pytest.mark.gpu

_up, _sz, _u, _f = ctypes.c_uint64, ctypes.c_size_t, ctypes.c_uint, ctypes.c_float


@pytest.fixture(scope="module")
def env():
    rt, kern = Runtime(), Kernels()
    L = kern.lib
    L.nya_hip_step.argtypes = [_up, _u, _sz, _up]
    L.nya_hip_embed.argtypes = [_up, _u, _sz, _sz, _up, _sz, _up, _f, _up]
    L.nya_hip_rms_norm.argtypes = [_up, _up, _up, _up, _sz, _sz, _f, _up]
    L.nya_hip_rope_qkv.argtypes = [_up, _sz, _up, _sz, _up, _sz, _sz, _sz, _sz, _sz, _up, _up, _sz, _up, _up, _up]
    L.nya_hip_attention.argtypes = [_up, _sz, _up, _up, _up, _up, _up, _sz, _sz, _sz, _sz, _sz, _sz, _f, _up]
    L.nya_hip_attention_split.argtypes = [_up, _sz, _up, _up, _up, _up, _up, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _f,
                                          _up]
    L.nya_hip_post_norm.argtypes = [_up, _up, _up, _f, _up, _up, _sz, _sz, _f, _up]
    L.nya_hip_head_norm_rope.argtypes = [_up, _sz, _up, _sz, _up, _sz, _sz, _sz, _sz, _sz, _up, _up, _f, _up, _up,
                                         _sz, _up, _up, _up]
    L.nya_hip_gelu_mul.argtypes = [_up, _sz, _up, _sz, _up, _sz, _sz, _up]
    L.nya_hip_matvec_geglu.argtypes = [_up, _u, _sz, _sz, _up, _up, _up]
    L.nya_hip_gelu_pairs.argtypes = [_up, _up, _sz, _sz, _up]
    L.nya_hip_softcap.argtypes = [_up, _sz, _f, _up]
    L.nya_hip_silu_mul.argtypes = [_up, _sz, _up, _sz, _up, _sz, _sz, _up]
    L.nya_hip_matvec_gated.argtypes = [_up, _u, _sz, _sz, _up, _up, _up, _up]
    L.nya_hip_matvec_swiglu.argtypes = [_up, _u, _sz, _sz, _up, _up, _up]
    L.nya_hip_matvec_residual.argtypes = [_up, _u, _sz, _sz, _up, _up, _up, _up, _up, _up]
    L.nya_hip_matvec_swiglu_scaled.argtypes = [_up, _u, _sz, _sz, _up, _up, _f, _up, _up]
    L.nya_hip_matvec_normed.argtypes = [_up, _u, _sz, _sz, _up, _up, _up, _f, _up, _up, _up]
    L.nya_hip_matvec_normed_rope.argtypes = [_up, _u, _sz, _sz, _sz, _up, _up, _up, _f, _up, _up, _up, _up, _sz,
                                             _sz, _sz, _sz, _up, _up, _up]
    L.nya_hip_silu_pairs.argtypes = [_up, _up, _sz, _sz, _up]
    L.nya_hip_matvec_scaled_rope.argtypes = [_up, _u, _sz, _sz, _sz, _up, _up, _f, _up, _up, _up, _sz, _sz, _sz,
                                             _sz, _up, _up, _up]
    L.nya_hip_matvec_rope_pair.argtypes = [_up, _u, _sz, _up, _u, _sz, _sz, _up, _up, _up, _up, _up, _f, _up, _up, _up,
                                           _sz, _sz, _sz, _sz, _up, _up, _up]
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


def test_step_slot(env):
    rt, L, stream = env
    dev = Dev(rt)
    try:
        slot = dev.empty(8)
        assert L.nya_hip_step(slot, 31999, 1234, stream) == 0
        rt.sync(stream)
        assert dev.get(slot, np.empty(2, np.uint32)).tolist() == [31999, 1234]
        assert L.nya_hip_step(slot + 2, 1, 0, stream) == 1   # misaligned
    finally:
        dev.close()


@pytest.mark.parametrize("type_id", [F32, F16, BF16, Q8_0, Q4_0, Q4_K, Q6_K])
@pytest.mark.parametrize("scale", [1.0, float(np.sqrt(np.float32(512)))], ids=["plain", "gemma"])
def test_embed_exact(env, oracle, type_id, scale):
    """The decoded rows, times Gemma's sqrt(d) (the engine's float
    product, backend/core/llm_cpu.c:453) where asked: bit for bit."""
    rt, L, stream = env
    rows, cols = 7, 512
    w = synth.weights(type_id, rows, cols, seed=40 + type_id)
    ref = oracle.dequant(w, type_id, rows, cols).reshape(rows, cols) * np.float32(scale)
    tokens = np.array([3, 0, rows - 1, rows + 5, 3], np.uint32)   # one id past the matrix
    dev = Dev(rt)
    try:
        wd, td, out = dev.put(w), dev.put(tokens), dev.empty(4 * cols * len(tokens))
        assert L.nya_hip_embed(wd, type_id, rows, cols, td, len(tokens), out, scale, stream) == 0
        rt.sync(stream)
        got = dev.get(out, np.empty((len(tokens), cols), np.float32))
        for i, t in enumerate(tokens):
            want = ref[t] if t < rows else np.zeros(cols, np.float32)
            assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32)), f"token {i} (id {t})"
        assert L.nya_hip_embed(wd, type_id, rows, cols, td, 0, out, 1.0, stream) == 1      # no tokens
        assert L.nya_hip_embed(wd, type_id, rows, cols, td, 1, out, float("inf"), stream) == 1
    finally:
        dev.close()


@pytest.mark.parametrize("n,offset", [(4096, 0), (2048, 0), (4098, 0), (4096, 4), (16384, 0)],
                         ids=["vector", "half", "ragged", "misaligned", "wide"])
@pytest.mark.parametrize("residual", [False, True])
def test_rms_norm(env, n, offset, residual):
    rt, L, stream = env
    count = 3
    rng = np.random.default_rng(n + offset)
    x = rng.standard_normal((count, n)).astype(np.float32)
    r = rng.standard_normal((count, n)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    eps = 1e-5
    xs32 = (x + r if residual else x).astype(np.float32)
    xs = xs32.astype(np.float64)
    scale = 1.0 / np.sqrt(np.sum(xs * xs, axis=1, keepdims=True) / n + eps)
    ref = xs * scale.astype(np.float32) * w
    dev = Dev(rt)
    try:
        xd, rd, wd, od = dev.put(x, offset), dev.put(r, offset), dev.put(w), dev.empty(4 * n * count)
        assert L.nya_hip_rms_norm(xd, rd if residual else 0, wd, od, n, count, eps, stream) == 0
        rt.sync(stream)
        assert scaled_error(dev.get(od, x), ref) <= 2e-6
        assert np.array_equal(dev.get(xd, x), xs32)      # the residual add written back (or x untouched)
    finally:
        dev.close()


def rotate(v, c, s, pairs):
    v = v.reshape(-1, pairs, 2).astype(np.float64)
    a, b = v[..., 0], v[..., 1]
    return np.stack([a * c - b * s, a * s + b * c], -1).reshape(-1)


@pytest.mark.parametrize("layout", ["fused", "split"])
@pytest.mark.parametrize("heads,kv_heads,width", [(32, 8, 128), (4, 4, 64), (6, 2, 80)])
def test_rope_qkv(env, heads, kv_heads, width, layout):
    rt, L, stream = env
    count, capacity = 4, 2000
    positions = np.array([1234, 1235, 1236, capacity + 3], np.int32)   # the last is outside the cache
    qd, kvd = heads * width, kv_heads * width
    rng = np.random.default_rng(heads * width)
    pairs = width // 2
    freq = (10000.0 ** (-np.arange(pairs) / pairs)).astype(np.float32)
    if layout == "fused":
        rows = rng.standard_normal((count, qd + 2 * kvd)).astype(np.float32)
        qs = ks = vs = qd + 2 * kvd
        q_at, k_at, v_at = 0, qd, qd + kvd
        blocks = [rows]
    else:   # q in one block, k|v in another (types that differ)
        qb = rng.standard_normal((count, qd)).astype(np.float32)
        kvb = rng.standard_normal((count, 2 * kvd)).astype(np.float32)
        qs, ks, vs = qd, 2 * kvd, 2 * kvd
        blocks = [qb, kvb]
    keys0 = rng.standard_normal((capacity, kvd)).astype(np.float32)
    values0 = rng.standard_normal((capacity, kvd)).astype(np.float32)
    dev = Dev(rt)
    try:
        ptrs = [dev.put(b) for b in blocks]
        if layout == "fused":
            q, k, v = ptrs[0] + 4 * q_at, ptrs[0] + 4 * k_at, ptrs[0] + 4 * v_at
        else:
            q, k, v = ptrs[0], ptrs[1], ptrs[1] + 4 * kvd
        fd, pd, kd, vd = dev.put(freq), dev.put(positions), dev.put(keys0), dev.put(values0)
        assert L.nya_hip_rope_qkv(q, qs, k, ks, v, vs, count, heads, kv_heads, width, fd, pd, capacity, kd, vd,
                                  stream) == 0
        rt.sync(stream)
        got = [dev.get(p, b) for p, b in zip(ptrs, blocks)]
        keys, values = dev.get(kd, keys0), dev.get(vd, values0)
        for i, pos in enumerate(positions):
            if layout == "fused":
                qin, kin, vin = blocks[0][i, :qd], blocks[0][i, qd:qd + kvd], blocks[0][i, qd + kvd:]
                qout, kvout = got[0][i, :qd], got[0][i, qd:]
            else:
                qin, kin, vin = blocks[0][i], blocks[1][i, :kvd], blocks[1][i, kvd:]
                qout, kvout = got[0][i], got[1][i]
            assert np.array_equal(kvout, np.concatenate([kin, vin]))          # k and v rows left in place
            if pos >= capacity:
                assert np.array_equal(qout, qin)
                continue
            angle = (np.float32(pos) * freq).astype(np.float64)
            c, s = np.cos(angle), np.sin(angle)
            assert scaled_error(qout, rotate(qin, c, s, pairs)) <= 2e-6
            assert scaled_error(keys[pos], rotate(kin, c, s, pairs)) <= 2e-6
            assert np.array_equal(values[pos], vin)
        untouched = np.setdiff1d(np.arange(capacity), positions[positions < capacity])
        assert np.array_equal(keys[untouched], keys0[untouched])
        assert np.array_equal(values[untouched], values0[untouched])
    finally:
        dev.close()


def attention_ref(q, keys, values, heads, kv_heads, width, length, scale, window=0):
    """Positions [0, length), the last `window` of them when window > 0."""
    first = length - window if 0 < window < length else 0
    q = q.reshape(heads, width).astype(np.float64)
    k = keys[first:length].reshape(length - first, kv_heads, width).astype(np.float64)
    v = values[first:length].reshape(length - first, kv_heads, width).astype(np.float64)
    group = heads // kv_heads
    out = np.empty((heads, width))
    for h in range(heads):
        s = k[:, h // group, :] @ q[h] * scale
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ v[:, h // group, :]
    return out.reshape(-1)


@pytest.mark.parametrize("heads,kv_heads,width,length,count,window", [
    (32, 8, 128, 1, 1, 0), (32, 8, 128, 37, 1, 0), (32, 8, 128, 1000, 1, 0), (8, 8, 64, 300, 1, 0),
    (6, 2, 80, 129, 1, 0), (4, 1, 256, 513, 1, 0), (8, 2, 128, 8192, 1, 0), (8, 2, 128, 9000, 1, 0),
    (32, 4, 64, 64, 64, 0), (8, 2, 128, 300, 5, 0), (6, 2, 80, 40, 7, 0), (4, 2, 128, 8300, 3, 0),
    (8, 2, 128, 1000, 1, 64), (4, 1, 256, 513, 3, 100), (6, 2, 80, 129, 7, 20), (8, 4, 64, 40, 12, 32),
    (8, 2, 128, 9000, 2, 4096), (8, 2, 128, 30, 4, 512),
    (8, 4, 512, 700, 1, 0), (4, 2, 512, 300, 6, 64), (4, 1, 320, 257, 3, 0), (2, 2, 512, 9000, 1, 1024),
])
def test_attention(env, heads, kv_heads, width, length, count, window):
    """`count` causal queries ending at position length - 1, the query rows
    strided past the fused k|v part as in the plan's buffers; with a window,
    each query attends its last `window` positions (a sliding layer)."""
    rt, L, stream = env
    rng = np.random.default_rng(length * 7 + width + count)
    max_length = length + 5
    q_stride = (heads + 2 * kv_heads) * width
    q = rng.standard_normal((count, q_stride)).astype(np.float32)
    keys = rng.standard_normal((max_length, kv_heads * width)).astype(np.float32)
    values = rng.standard_normal((max_length, kv_heads * width)).astype(np.float32)
    positions = np.arange(length - count, length, dtype=np.int32)
    scale = float(1 / np.sqrt(np.float32(width)))
    ref = np.concatenate([attention_ref(q[i, :heads * width], keys, values, heads, kv_heads, width, int(p) + 1,
                                        np.float32(scale), window) for i, p in enumerate(positions)])
    dev = Dev(rt)
    try:
        qd, kd, vd, pd = dev.put(q), dev.put(keys), dev.put(values), dev.put(positions)
        od = dev.empty(4 * count * heads * width)
        sd = dev.empty(4 * count * heads * max_length) if max_length > 8192 else 0
        assert L.nya_hip_attention(qd, q_stride, kd, vd, od, sd, pd, count, heads, kv_heads, width, max_length,
                                   window, scale, stream) == 0
        rt.sync(stream)
        err = scaled_error(dev.get(od, np.empty(count * heads * width, np.float32)), ref)
        print(f"attention {heads}/{kv_heads} x {width}, length {length}, {count} queries, window {window}: "
              f"scaled error {err:.3g}", flush=True)
        assert err <= 1e-5
    finally:
        dev.close()


@pytest.mark.parametrize("heads,kv_heads,width,length,count,window", [
    (32, 8, 128, 1, 1, 0), (32, 8, 128, 37, 3, 0), (8, 8, 64, 5, 2, 0), (4, 1, 256, 20, 1, 0),
    (4, 2, 512, 9, 2, 0), (32, 8, 128, 200, 1, 0), (32, 8, 128, 37, 3, 64), (8, 4, 128, 150, 3, 40),
    (4, 2, 256, 90, 2, 16), (4, 2, 512, 30, 2, 8),
])
def test_attention_ignores_rows_past_the_range(env, heads, kv_heads, width, length, count, window):
    """The kernel requests the first key and value rows from row 0 before it
    reads the position (and again from the window's start once a window has
    moved on): rows of the cache outside the causal range (here NaN and
    infinities, before a window and past the range, up to max_length) never
    reach the output. A query with position -1 leaves its output as it was."""
    rt, L, stream = env
    rng = np.random.default_rng(length + width)
    max_length = 256
    q_stride = (heads + 2 * kv_heads) * width
    count += 1   # query 0 has no causal range at all
    q = rng.standard_normal((count, q_stride)).astype(np.float32)
    keys = rng.standard_normal((max_length, kv_heads * width)).astype(np.float32)
    values = rng.standard_normal((max_length, kv_heads * width)).astype(np.float32)
    positions = np.concatenate([[-1], np.arange(length - count + 1, length)]).astype(np.int32)
    keys[length:] = np.nan
    values[length:] = np.nan
    values[length::3] = np.inf
    if window:
        # Before the earliest query's window.
        before = max(0, int(positions[1]) + 1 - window)
        keys[:before] = np.nan
        values[:before] = -np.inf
    scale = float(1 / np.sqrt(np.float32(width)))
    sentinel = np.full(heads * width, 7.0, np.float32)
    dev = Dev(rt)
    try:
        qd, kd, vd, pd = dev.put(q), dev.put(keys), dev.put(values), dev.put(positions)
        od = dev.put(np.tile(sentinel, count))
        assert L.nya_hip_attention(qd, q_stride, kd, vd, od, 0, pd, count, heads, kv_heads, width, max_length,
                                   window, scale, stream) == 0
        rt.sync(stream)
        got = dev.get(od, np.empty(count * heads * width, np.float32)).reshape(count, -1)
        assert np.array_equal(got[0], sentinel)
        for i in range(1, count):
            ref = attention_ref(q[i, :heads * width], keys, values, heads, kv_heads, width, int(positions[i]) + 1,
                                np.float32(scale), window)
            assert np.all(np.isfinite(got[i]))
            assert scaled_error(got[i], ref) <= 1e-5
    finally:
        dev.close()


SPLIT_CASES = [(32, 8, 128, 4096, 1, 64, 0), (32, 4, 64, 1000, 1, 16, 0), (8, 8, 128, 300, 1, 8, 0),
               (16, 8, 128, 2000, 3, 32, 0), (8, 2, 256, 5000, 2, 8, 0), (32, 4, 64, 20000, 1, 32, 0),
               (32, 8, 128, 5, 1, 64, 0), (32, 8, 128, 257, 33, 8, 0), (8, 2, 128, 600, 2, 300, 0),
               (32, 8, 128, 4096, 1, 64, 1024), (8, 2, 256, 5000, 2, 8, 700), (16, 8, 128, 2000, 33, 32, 100),
               (2, 2, 512, 5000, 2, 8, 0), (8, 4, 512, 2000, 3, 64, 512), (4, 2, 512, 3000, 1, 300, 0)]


@pytest.mark.parametrize("heads,kv_heads,width,length,count,splits,window", SPLIT_CASES,
                         ids=[f"{h}/{k}x{w}-len{n}-q{c}-s{s}-w{win}" for h, k, w, n, c, s, win in SPLIT_CASES])
def test_attention_split(env, heads, kv_heads, width, length, count, splits, window):
    """The attention split over the cached positions (every query head of a
    KV head per workgroup, then the combination of the partial softmaxes):
    against the float64 statement of the engine's step, and beside the
    one-workgroup-per-head kernel; more splits than positions leave empty
    partials; a window splits only the positions it keeps."""
    rt, L, stream = env
    rng = np.random.default_rng(length * 11 + width + count + splits)
    max_length = length + 3
    q_stride = (heads + 2 * kv_heads) * width
    q = rng.standard_normal((count, q_stride)).astype(np.float32)
    keys = rng.standard_normal((max_length, kv_heads * width)).astype(np.float32)
    values = rng.standard_normal((max_length, kv_heads * width)).astype(np.float32)
    positions = np.arange(length - count, length, dtype=np.int32)
    scale = float(1 / np.sqrt(np.float32(width)))
    ref = np.concatenate([attention_ref(q[i, :heads * width], keys, values, heads, kv_heads, width, int(p) + 1,
                                        np.float32(scale), window) for i, p in enumerate(positions)])
    dev = Dev(rt)
    try:
        qd, kd, vd, pd = dev.put(q), dev.put(keys), dev.put(values), dev.put(positions)
        od, od2 = dev.empty(4 * count * heads * width), dev.empty(4 * count * heads * width)
        part = dev.empty(4 * count * heads * splits * (width + 2))
        sd = dev.empty(4 * count * heads * max_length) if max_length > 8192 else 0
        print(f"attention_split {heads}/{kv_heads} x {width}, length {length}, {count} queries, {splits} splits, "
              f"window {window}", flush=True)
        assert L.nya_hip_attention_split(qd, q_stride, kd, vd, od, part, pd, count, heads, kv_heads, width,
                                         max_length, window, splits, scale, stream) == 0
        assert L.nya_hip_attention(qd, q_stride, kd, vd, od2, sd, pd, count, heads, kv_heads, width, max_length,
                                   window, scale, stream) == 0
        rt.sync(stream)
        got = dev.get(od, np.empty(count * heads * width, np.float32))
        err = scaled_error(got, ref)
        err2 = scaled_error(got, dev.get(od2, np.empty(count * heads * width, np.float32)).astype(np.float64))
        print(f"  scaled error {err:.3g} (against the unsplit kernel {err2:.3g})", flush=True)
        assert err <= 1e-5 and err2 <= 1e-5
    finally:
        dev.close()


def test_attention_split_declines(env):
    rt, L, stream = env
    dev = Dev(rt)
    try:
        p = dev.empty(4 * 4096)
        args = lambda heads, kv, width, max_length, splits: (p, (heads + 2 * kv) * width, p, p, p, p, p, 1, heads, kv,
                                                            width, max_length, 0, splits, 1.0, stream)
        assert L.nya_hip_attention_split(*args(32, 8, 80, 1000, 8)) == 1      # width 80
        assert L.nya_hip_attention_split(*args(48, 3, 128, 1000, 8)) == 1     # 16 query heads per KV head
        assert L.nya_hip_attention_split(*args(32, 4, 256, 1000, 8)) == 1     # 8 heads of width 256
        assert L.nya_hip_attention_split(*args(32, 8, 128, 9000, 8)) == 1     # 1125 positions per split
        assert L.nya_hip_attention_split(*args(16, 4, 512, 1000, 8)) == 1     # 4 heads of width 512
        assert L.nya_hip_attention_split(p + 4, 384, p, p, p, p, p, 1, 2, 1, 128, 100, 0, 4, 1.0, stream) == 1  # q align
    finally:
        dev.close()


def test_attention_declines(env):
    rt, L, stream = env
    dev = Dev(rt)
    try:
        p = dev.empty(4 * 4 * 512)
        assert L.nya_hip_attention(p, 2048, p, p, p, p, p, 1, 2, 2, 1024, 1, 0, 1.0, stream) == 1   # width > 512
        assert L.nya_hip_attention(p, 256, p, p, p, 0, p, 1, 2, 2, 128, 9000, 0, 1.0, stream) == 1  # scratch needed
    finally:
        dev.close()


@pytest.mark.parametrize("layout", ["fused", "split", "in-place"])
def test_silu_mul(env, layout):
    rt, L, stream = env
    rng = np.random.default_rng(5)
    n = 14336
    count = 1 if layout == "in-place" else 3
    g = (4 * rng.standard_normal((count, n))).astype(np.float32)
    u = rng.standard_normal((count, n)).astype(np.float32)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    dev = Dev(rt)
    try:
        if layout == "split":
            gd, ud = dev.put(g), dev.put(u)
            gs = us = n
        else:
            gu = dev.put(np.concatenate([g, u], axis=1))
            gd, ud, gs, us = gu, gu + 4 * n, 2 * n, 2 * n
        out = gd if layout == "in-place" else dev.empty(4 * n * count)
        assert L.nya_hip_silu_mul(gd, gs, ud, us, out, n, count, stream) == 0
        rt.sync(stream)
        assert scaled_error(dev.get(out, g), ref) <= 2e-6
        if layout != "in-place":
            assert L.nya_hip_silu_mul(gd, gs, ud, us, gd, n, count, stream) == 1   # overlapping output
    finally:
        dev.close()


def norm32(x, w, eps):
    """The engine's RMS norm of each row (backend/core/llm_cpu.c:83-104) in
    float32 steps: the sum of squares in double, its scale rounded to
    float32, then x * scale * w."""
    x = np.asarray(x, np.float32)
    scale = (1.0 / np.sqrt(np.sum(x.astype(np.float64) ** 2, axis=-1, keepdims=True) / x.shape[-1] +
                           np.float64(np.float32(eps)))).astype(np.float32)
    y = x * scale
    return y * w if w is not None else y


@pytest.mark.parametrize("n", [640, 1000, 2560, 5376, 16384])
@pytest.mark.parametrize("form", ["post", "plain", "no-residual"])
def test_post_norm(env, n, form):
    """Gemma's residual add through the branch's post norm, the block's
    output scale, then the next norm (backend/core/llm_cpu.c:514-515,
    :531-547): x written back and out against the engine's float32 steps;
    without a post weight the plain add, without a residual only the scale
    and the norm."""
    rt, L, stream = env
    count, eps, oscale = 3, 1e-6, np.float32(0.8125)
    rng = np.random.default_rng(n)
    x = rng.standard_normal((count, n)).astype(np.float32)
    r = (3 * rng.standard_normal((count, n))).astype(np.float32)
    post = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    if form == "post":
        xs = ((x + norm32(r, post, eps)) * oscale).astype(np.float32)
    elif form == "plain":
        xs = ((x + r) * oscale).astype(np.float32)
    else:
        xs = (x * oscale).astype(np.float32)
    ref = norm32(xs, w, eps)
    dev = Dev(rt)
    try:
        xd, rd, pd, wd, od = dev.put(x), dev.put(r), dev.put(post), dev.put(w), dev.empty(4 * n * count)
        rarg, parg = (rd, pd) if form == "post" else (rd, 0) if form == "plain" else (0, 0)
        assert L.nya_hip_post_norm(xd, rarg, parg, float(oscale), wd, od, n, count, eps, stream) == 0
        rt.sync(stream)
        assert scaled_error(dev.get(xd, x), xs.astype(np.float64)) <= 2e-6
        assert scaled_error(dev.get(od, x), ref.astype(np.float64)) <= 2e-6
        assert np.array_equal(dev.get(rd, r), r)      # the branch output is read, not written
        assert L.nya_hip_post_norm(xd, 0, pd, 1.0, wd, od, n, count, eps, stream) == 1       # post without residual
        assert L.nya_hip_post_norm(xd, rd, pd, 1.0, wd, od, 16385, 1, eps, stream) == 1      # wider than 16384
    finally:
        dev.close()


def rotate_halves(v, c, s):
    """Gemma's rotation of one head (backend/core/llm_cpu.c:345-358)."""
    half = v.shape[-1] // 2
    a, b = v[..., :half].astype(np.float64), v[..., half:].astype(np.float64)
    return np.concatenate([a * c - b * s, b * c + a * s], -1)


@pytest.mark.parametrize("heads,kv_heads,width", [(8, 4, 256), (4, 2, 128), (6, 2, 80), (2, 1, 64), (4, 2, 512),
                                                  (2, 1, 320)])
@pytest.mark.parametrize("form", ["qkv", "key-as-value", "q-only"])
def test_head_norm_rope(env, heads, kv_heads, width, form):
    """The Gemma q/k/v step: per-head norms (q and k weighted, v without a
    weight), the half-split rotation of q (in place) and k (into its cache
    slot), v into its slot; a key projection standing in for the value; a
    layer reading another's cache (q only); a position outside the cache
    leaves everything alone."""
    rt, L, stream = env
    count, capacity, eps = 4, 300, 1e-6
    positions = np.array([17, 18, 250, capacity + 1], np.int32)
    qd, kvd, half = heads * width, kv_heads * width, width // 2
    rng = np.random.default_rng(heads * width + len(form))
    stride = qd + 2 * kvd
    rows = (2 * rng.standard_normal((count, stride))).astype(np.float32)
    q_norm = (1 + 0.1 * rng.standard_normal(width)).astype(np.float32)
    k_norm = (1 + 0.1 * rng.standard_normal(width)).astype(np.float32)
    freq = (10000.0 ** (-np.arange(half) / half)).astype(np.float32)
    keys0 = rng.standard_normal((capacity, kvd)).astype(np.float32)
    values0 = rng.standard_normal((capacity, kvd)).astype(np.float32)
    dev = Dev(rt)
    try:
        rd, qn, kn, fd, pd = dev.put(rows), dev.put(q_norm), dev.put(k_norm), dev.put(freq), dev.put(positions)
        kd, vd = dev.put(keys0), dev.put(values0)
        k_at = rd + 4 * qd
        v_at = k_at if form == "key-as-value" else rd + 4 * (qd + kvd)
        kp = 0 if form == "q-only" else k_at
        print(f"head_norm_rope {heads}/{kv_heads} x {width}, {form}", flush=True)
        assert L.nya_hip_head_norm_rope(rd, stride, kp, stride, v_at, stride, count, heads, kv_heads, width, qn, kn,
                                        eps, fd, pd, capacity, kd, vd, stream) == 0
        rt.sync(stream)
        got = dev.get(rd, rows)
        keys, values = dev.get(kd, keys0), dev.get(vd, values0)
        for i, pos in enumerate(positions):
            if pos >= capacity:
                assert np.array_equal(got[i], rows[i])
                continue
            angle = (np.float32(pos) * freq).astype(np.float64)
            c, s = np.cos(angle), np.sin(angle)
            q = norm32(rows[i, :qd].reshape(heads, width), q_norm, eps)
            assert scaled_error(got[i, :qd], rotate_halves(q, c, s).reshape(-1)) <= 2e-6
            assert np.array_equal(got[i, qd:], rows[i, qd:])   # k and v rows are read, not written
            if form == "q-only":
                continue
            k = norm32(rows[i, qd:qd + kvd].reshape(kv_heads, width), k_norm, eps)
            v_src = rows[i, qd:qd + kvd] if form == "key-as-value" else rows[i, qd + kvd:]
            v = norm32(v_src.reshape(kv_heads, width), None, eps)
            assert scaled_error(keys[pos], rotate_halves(k, c, s).reshape(-1)) <= 2e-6
            assert scaled_error(values[pos], v.reshape(-1).astype(np.float64)) <= 2e-6
        touched = positions[positions < capacity] if form != "q-only" else np.array([], np.int32)
        untouched = np.setdiff1d(np.arange(capacity), touched)
        assert np.array_equal(keys[untouched], keys0[untouched])
        assert np.array_equal(values[untouched], values0[untouched])
        assert L.nya_hip_head_norm_rope(rd, stride, kp, stride, v_at, stride, count, heads, kv_heads, 514, qn, kn,
                                        eps, fd, pd, capacity, kd, vd, stream) == 1    # wider than 512
    finally:
        dev.close()


@pytest.mark.parametrize("layout", ["fused", "split", "in-place"])
def test_gelu_mul(env, layout):
    """Gemma's gate (backend/core/llm_cpu.c:329-341) against float64."""
    rt, L, stream = env
    rng = np.random.default_rng(6)
    n = 10240 if layout != "split" else 1001
    count = 1 if layout == "in-place" else 3
    g = (4 * rng.standard_normal((count, n))).astype(np.float32)
    u = rng.standard_normal((count, n)).astype(np.float32)
    x = g.astype(np.float64)
    ref = 0.5 * x * (1 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3))) * u
    dev = Dev(rt)
    try:
        if layout == "split":
            gd, ud = dev.put(g), dev.put(u)
            gs = us = n
        else:
            gu = dev.put(np.concatenate([g, u], axis=1))
            gd, ud, gs, us = gu, gu + 4 * n, 2 * n, 2 * n
        out = gd if layout == "in-place" else dev.empty(4 * n * count)
        assert L.nya_hip_gelu_mul(gd, gs, ud, us, out, n, count, stream) == 0
        rt.sync(stream)
        assert scaled_error(dev.get(out, g), ref) <= 2e-6
        if layout != "in-place":
            assert L.nya_hip_gelu_mul(gd, gs, ud, us, gd, n, count, stream) == 1   # overlapping output
    finally:
        dev.close()


def test_softcap(env):
    """The final soft cap (backend/core/llm_cpu.c:562-565) against float64."""
    rt, L, stream = env
    rng = np.random.default_rng(8)
    x = (40 * rng.standard_normal(3 * 262144 + 5)).astype(np.float32)
    cap = 30.0
    ref = cap * np.tanh(x.astype(np.float64) / cap)
    dev = Dev(rt)
    try:
        xd = dev.put(x)
        assert L.nya_hip_softcap(xd, x.size, cap, stream) == 0
        rt.sync(stream)
        assert scaled_error(dev.get(xd, x), ref) <= 2e-6
        assert L.nya_hip_softcap(xd, x.size, 0.0, stream) == 1
    finally:
        dev.close()


@pytest.mark.parametrize("t,rows,cols", [(Q6_K, 4096, 14336), (Q4_K, 4096, 14336), (Q6_K, 2048, 5632),
                                         (Q4_0, 4096, 11008), (Q8_0, 1000, 4096), (Q4_K, 8192, 28672),
                                         (Q6_K, 300, 256)])
def test_matvec_gated_equals_two_steps(env, t, rows, cols):
    rt, L, stream = env
    kern = Kernels()
    rng = np.random.default_rng(rows + cols)
    g = (4 * rng.standard_normal(cols)).astype(np.float32)
    u = rng.standard_normal(cols).astype(np.float32)
    w = kern.device_weights(synth.weights(t, rows, cols, seed=rows), t, rows, cols)
    dev = Dev(rt)
    try:
        wd, gd, ud = dev.put(w), dev.put(g), dev.put(u)
        v, y1, y2 = dev.empty(4 * cols), dev.empty(4 * rows), dev.empty(4 * rows)
        print(f"gated {t} {rows}x{cols}", flush=True)
        assert L.nya_hip_matvec_gated(wd, t, rows, cols, gd, ud, y1, stream) == 0
        assert L.nya_hip_silu_mul(gd, cols, ud, cols, v, cols, 1, stream) == 0
        kern.matmul(wd, t, rows, cols, v, y2, 1, 0, 0, stream)
        rt.sync(stream)
        a, b = dev.get(y1, np.empty(rows, np.float32)), dev.get(y2, np.empty(rows, np.float32))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    finally:
        dev.close()


def test_matvec_gated_declines(env):
    rt, L, stream = env
    dev = Dev(rt)
    try:
        p = dev.empty(4 * 8192)
        assert L.nya_hip_matvec_gated(p, F16, 64, 256, p, p, p, stream) == 1          # dense type
        assert L.nya_hip_matvec_gated(p, Q4_0, 64, 288, p, p, p, stream) == 1         # short last group
        assert L.nya_hip_matvec_gated(p, Q4_K, 20480, 256, p, p, p, stream) == 1      # > 64 rows per CU
        assert L.nya_hip_matvec_gated(p, Q4_K, 64, 256, p + 4, p, p, stream) == 1     # gate not 16-byte aligned
    finally:
        dev.close()


@pytest.mark.parametrize("rows,cols", [(28672, 4096), (17408, 256), (22528, 2048), (11264, 2048)])
def test_matvec_swiglu_equals_two_steps(env, rows, cols):
    rt, L, stream = env
    kern = Kernels()
    assert L.nya_hip_matvec_swiglu(0, Q4_K, rows, cols, 0, 0, stream) == 0
    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal(cols).astype(np.float32)
    w = kern.device_weights(synth.weights(Q4_K, rows, cols, seed=rows), Q4_K, rows, cols)
    dev = Dev(rt)
    try:
        wd, xd = dev.put(w), dev.put(x)
        y, h1, h2 = dev.empty(4 * rows), dev.empty(2 * rows), dev.empty(2 * rows)
        print(f"swiglu {rows}x{cols}", flush=True)
        assert L.nya_hip_matvec_swiglu(wd, Q4_K, rows, cols, xd, h1, stream) == 0
        kern.matmul(wd, Q4_K, rows, cols, xd, y, 1, 0, 0, stream)
        assert L.nya_hip_silu_pairs(y, h2, rows // 2, 1, stream) == 0
        rt.sync(stream)
        a, b = dev.get(h1, np.empty(rows // 2, np.float32)), dev.get(h2, np.empty(rows // 2, np.float32))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        yv = dev.get(y, np.empty(rows, np.float32)).astype(np.float64).reshape(-1, 2, 16)
        g, u = yv[:, 0, :].reshape(-1), yv[:, 1, :].reshape(-1)
        assert scaled_error(b, g / (1 + np.exp(-g)) * u) <= 2e-6
    finally:
        dev.close()


@pytest.mark.parametrize("rows,cols", [(30720, 3840), (17408, 256), (11264, 2048)])
def test_matvec_geglu_equals_two_steps(env, rows, cols):
    """Gemma's gate|up product with the GELU gate in its epilogue: bit for
    bit the product followed by nya_hip_gelu_pairs, which meets the float64
    gate; several tokens through nya_hip_gelu_pairs."""
    rt, L, stream = env
    kern = Kernels()
    assert L.nya_hip_matvec_geglu(0, Q4_K, rows, cols, 0, 0, stream) == 0
    rng = np.random.default_rng(rows + cols + 1)
    x = rng.standard_normal(cols).astype(np.float32)
    w = kern.device_weights(synth.weights(Q4_K, rows, cols, seed=rows + 1), Q4_K, rows, cols)
    dev = Dev(rt)
    try:
        wd, xd = dev.put(w), dev.put(x)
        y, h1, h2 = dev.empty(4 * rows), dev.empty(2 * rows), dev.empty(2 * rows)
        print(f"geglu {rows}x{cols}", flush=True)
        assert L.nya_hip_matvec_geglu(wd, Q4_K, rows, cols, xd, h1, stream) == 0
        kern.matmul(wd, Q4_K, rows, cols, xd, y, 1, 0, 0, stream)
        assert L.nya_hip_gelu_pairs(y, h2, rows // 2, 1, stream) == 0
        rt.sync(stream)
        a, b = dev.get(h1, np.empty(rows // 2, np.float32)), dev.get(h2, np.empty(rows // 2, np.float32))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        yv = dev.get(y, np.empty(rows, np.float32)).astype(np.float64).reshape(-1, 2, 16)
        g, u = yv[:, 0, :].reshape(-1), yv[:, 1, :].reshape(-1)
        assert scaled_error(b, 0.5 * g * (1 + np.tanh(0.7978845608028654 * (g + 0.044715 * g ** 3))) * u) <= 2e-6
        assert L.nya_hip_matvec_geglu(0, Q6_K, rows, cols, 0, 0, stream) == 1    # Q4_K only, as SwiGLU
        assert L.nya_hip_gelu_pairs(y, y, rows // 2, 1, stream) == 1             # overlapping
    finally:
        dev.close()


def test_matvec_swiglu_declines(env):
    rt, L, stream = env
    assert L.nya_hip_matvec_swiglu(0, Q4_K, 8192, 4096, 0, 0, stream) == 1     # 32 rows per CU: the row kernel
    assert L.nya_hip_matvec_swiglu(0, Q6_K, 28672, 4096, 0, 0, stream) == 1    # not Q4_K
    assert L.nya_hip_matvec_swiglu(0, Q4_K, 28672, 20480, 0, 0, stream) == 1   # more than one column chunk
    assert L.nya_hip_matvec_swiglu(0, Q4_K, 28688, 4096, 0, 0, stream) == 1    # not whole 32-row blocks


NORM_PARTS = 256


@pytest.mark.parametrize("t,rows,cols", [(Q4_K, 4096, 4096), (Q4_K, 2048, 2048), (Q6_K, 4096, 4096),
                                         (Q8_0, 1000, 4096), (Q4_0, 8192, 1024), (Q4_K, 16384, 256),
                                         (Q6_K, 5010, 512)])
def test_matvec_residual(env, t, rows, cols):
    """The attention output product with the residual epilogue: res + W x in
    place equals the norm step's residual add of nya_hip_matmul's product bit
    for bit, hn = res * norm bit for bit, and partial sum j is the double sum
    of res^2 over workgroup j's rows (ceil(rows / 256) rows each on 256 CUs:
    16, 8, 4, 32, 64 and 20 rows; at 5010 rows the last of 251 workgroups
    holds 10, in a short last tile), zeros past the last workgroup."""
    rt, L, stream = env
    kern = Kernels()
    assert L.nya_hip_matvec_residual(0, t, rows, cols, 0, 0, 0, 0, 0, 0) == 0
    rng = np.random.default_rng(rows + 7 * cols + t)
    x = rng.standard_normal(cols).astype(np.float32)
    res = (2 * rng.standard_normal(rows)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(rows)).astype(np.float32)
    w = kern.device_weights(synth.weights(t, rows, cols, seed=rows + 2), t, rows, cols)
    dev = Dev(rt)
    try:
        wd, xd, r1, r2, gd = dev.put(w), dev.put(x), dev.put(res), dev.put(res), dev.put(g)
        hn, y, xn = dev.empty(4 * rows), dev.empty(4 * rows), dev.empty(4 * rows)
        parts = dev.put(np.full(NORM_PARTS, 7.0))   # stale values: every entry is written
        print(f"residual {TYPE_NAMES[t]} {rows}x{cols}", flush=True)
        assert L.nya_hip_matvec_residual(wd, t, rows, cols, xd, r1, gd, hn, parts, stream) == 0
        kern.matmul(wd, t, rows, cols, xd, y, 1, 0, 0, stream)
        assert L.nya_hip_rms_norm(r2, y, gd, xn, rows, 1, 1e-5, stream) == 0   # r2 += y in place
        rt.sync(stream)
        bits = lambda p, n: dev.get(p, np.empty(n, np.float32)).view(np.uint32)
        h = bits(r1, rows)
        assert np.array_equal(h, bits(r2, rows))
        hv = h.view(np.float32)
        assert np.array_equal(bits(hn, rows), (hv * g).view(np.uint32))
        ps = dev.get(parts, np.empty(NORM_PARTS, np.float64))
    finally:
        dev.close()
    rw = -(-rows // 256)
    wgs = -(-rows // rw)
    want = np.zeros(NORM_PARTS)
    hd = hv.astype(np.float64) ** 2
    for j in range(wgs):
        want[j] = hd[j * rw:(j + 1) * rw].sum()
    assert np.all(ps[wgs:] == 0.0)
    assert np.allclose(ps[:wgs], want[:wgs], rtol=1e-12, atol=0)


def test_matvec_residual_declines(env):
    rt, L, stream = env
    q = lambda t, rows, cols: L.nya_hip_matvec_residual(0, t, rows, cols, 0, 0, 0, 0, 0, 0)
    assert q(Q4_K, 16384, 4096) == 0      # 64 rows per CU
    assert q(Q4_K, 16385, 4096) == 1      # 65: three tiles per workgroup
    assert q(Q4_K, 4096, 20736) == 1      # two column chunks
    assert q(F16, 4096, 4096) == 1
    dev = Dev(rt)
    try:
        p = dev.empty(1 << 16)   # every call is refused before anything is enqueued
        assert L.nya_hip_matvec_residual(p, Q4_K, 4096, 4096, p, p, p, p, 0, stream) == 1           # no parts
        assert L.nya_hip_matvec_residual(p, Q4_K, 4096, 4096, p, p + 16384, p, p + 32768, p + 49156,
                                         stream) == 1                                                 # parts align
        assert L.nya_hip_matvec_residual(p, Q4_K, 4096, 4096, p, p, p, p + 64, p + 8, stream) == 1   # hn over x
    finally:
        dev.close()


@pytest.mark.parametrize("rows,cols", [(28672, 4096), (11264, 2048), (17408, 256), (22528, 3840)])
def test_matvec_swiglu_scaled(env, oracle, rows, cols):
    """The gate|up product of hn = h * g with the norm's scale from partial
    sums of squares (8B and TinyLlama shapes, one group, 15 of 16 groups):
    within the contract bound 1e-6 (1 + sum |w xn|) on each gate and up sum
    (backend/tests/test_quant_kernels.c:13-25) of the double-precision norm,
    carried through silu(g) u (|d/dg| <= 1.1 |u|, |d/du| = |silu(g)|), plus
    1e-6 of the value for the float SiLU; the norm step followed by
    nya_hip_matvec_swiglu meets the same bound."""
    rt, L, stream = env
    assert L.nya_hip_matvec_swiglu_scaled(0, Q4_K, rows, cols, 0, 0, 1e-5, 0, 0) == 0
    rng = np.random.default_rng(rows + cols + 3)
    h = (3 * rng.standard_normal(cols)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    hd = h.astype(np.float64)
    parts = np.zeros(NORM_PARTS)
    run = -(-cols // 200)
    for j in range(0, cols, run):
        parts[j // run] = float((hd[j:j + run] ** 2).sum())
    host = synth.weights(Q4_K, rows, cols, seed=rows + 1)
    w = Kernels().device_weights(host, Q4_K, rows, cols)
    dev = Dev(rt)
    try:
        wd, hnd, pd, xd, gd = dev.put(w), dev.put(h * g), dev.put(parts), dev.put(h), dev.put(g)
        xn, h1, h2 = dev.empty(4 * cols), dev.empty(2 * rows), dev.empty(2 * rows)
        print(f"swiglu scaled {rows}x{cols}", flush=True)
        assert L.nya_hip_matvec_swiglu_scaled(wd, Q4_K, rows, cols, hnd, pd, 1e-5, h1, stream) == 0
        assert L.nya_hip_rms_norm(xd, 0, gd, xn, cols, 1, 1e-5, stream) == 0
        assert L.nya_hip_matvec_swiglu(wd, Q4_K, rows, cols, xn, h2, stream) == 0
        rt.sync(stream)
        fused = dev.get(h1, np.empty(rows // 2, np.float32))
        steps = dev.get(h2, np.empty(rows // 2, np.float32))
    finally:
        dev.close()
    xnd = hd / np.sqrt(np.mean(hd * hd) + 1e-5) * g.astype(np.float64)
    sums, mags = oracle.contract_sums(host, Q4_K, xnd, rows, cols)
    pick = lambda a, half: a[0].reshape(-1, 2, 16)[:, half, :].reshape(-1)
    gs, us, gm, um = pick(sums, 0), pick(sums, 1), pick(mags, 0), pick(mags, 1)
    silu = gs / (1 + np.exp(-gs))
    want = silu * us
    bound = 1.1 * np.abs(us) * 1e-6 * (1 + gm) + np.abs(silu) * 1e-6 * (1 + um) + 1e-6 * np.abs(want)
    for name, got in (("scaled", fused), ("two steps", steps)):
        err = np.abs(got.astype(np.float64) - want)
        bad = ~np.isfinite(got) | (err > bound)
        assert not bad.any(), f"{name}: {int(bad.sum())} outside, worst {float((err / bound).max()):.3g} of the bound"
        print(f"  {name}: worst {float((err / bound).max()):.3g} of the bound", flush=True)


def test_matvec_swiglu_scaled_declines(env):
    rt, L, stream = env
    q = lambda t, rows, cols: L.nya_hip_matvec_swiglu_scaled(0, t, rows, cols, 0, 0, 1e-5, 0, 0)
    assert q(Q4_K, 28672, 4096) == 0
    assert q(Q4_K, 8192, 4096) == 1      # 32 rows per CU: not the gate|up kernel
    assert q(Q6_K, 28672, 4096) == 1
    dev = Dev(rt)
    try:
        p = dev.empty(1 << 16)   # every call is refused before anything is enqueued
        assert L.nya_hip_matvec_swiglu_scaled(p, Q4_K, 28672, 4096, p + 4, p, 1e-5, p, stream) == 1   # hn align
        assert L.nya_hip_matvec_swiglu_scaled(p, Q4_K, 28672, 4096, p, p + 4, 1e-5, p, stream) == 1   # parts align
        assert L.nya_hip_matvec_swiglu_scaled(p, Q4_K, 28672, 4096, p, 0, 1e-5, p, stream) == 1       # no parts
    finally:
        dev.close()


@pytest.mark.parametrize("t,rows,cols,residual", [(Q4_K, 6144, 4096, True), (Q4_K, 6144, 4096, False),
                                                  (Q6_K, 2560, 2048, True), (Q8_0, 1000, 4096, True),
                                                  (Q4_0, 3000, 1024, True), (Q4_K, 8192, 256, True)])
def test_matvec_normed_equals_two_steps(env, t, rows, cols, residual):
    rt, L, stream = env
    kern = Kernels()
    assert L.nya_hip_matvec_normed(0, t, rows, cols, 0, 0, 0, 1e-5, 0, 0, stream) == 0
    rng = np.random.default_rng(rows + cols)
    x = (3 * rng.standard_normal(cols)).astype(np.float32)
    r = rng.standard_normal(cols).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    w = kern.device_weights(synth.weights(t, rows, cols, seed=rows), t, rows, cols)
    dev = Dev(rt)
    try:
        wd, x1, x2, rd, gd = dev.put(w), dev.put(x), dev.put(x), dev.put(r), dev.put(g)
        hout, xn = dev.empty(4 * cols), dev.empty(4 * cols)
        y1, y2 = dev.empty(4 * rows), dev.empty(4 * rows)
        print(f"normed {t} {rows}x{cols} residual {residual}", flush=True)
        assert L.nya_hip_matvec_normed(wd, t, rows, cols, x1, rd if residual else 0, gd, 1e-5,
                                       hout if residual else 0, y1, stream) == 0
        assert L.nya_hip_rms_norm(x2, rd if residual else 0, gd, xn, cols, 1, 1e-5, stream) == 0
        kern.matmul(wd, t, rows, cols, xn, y2, 1, 0, 0, stream)
        rt.sync(stream)
        bits = lambda p, n: dev.get(p, np.empty(n, np.float32)).view(np.uint32)
        assert np.array_equal(bits(y1, rows), bits(y2, rows))
        if residual:
            assert np.array_equal(bits(hout, cols), bits(x2, cols))   # the norm step's in-place residual
        assert np.array_equal(bits(x1, cols), x.view(np.uint32))      # x itself untouched
    finally:
        dev.close()


def test_matvec_normed_declines(env):
    rt, L, stream = env
    assert L.nya_hip_matvec_normed(0, Q4_K, 14336, 4096, 0, 0, 0, 1e-5, 0, 0, stream) == 1   # 56 rows per CU
    assert L.nya_hip_matvec_normed(0, Q4_K, 4096, 8192, 0, 0, 0, 1e-5, 0, 0, stream) == 1    # 8192 columns
    assert L.nya_hip_matvec_normed(0, F16, 4096, 4096, 0, 0, 0, 1e-5, 0, 0, stream) == 1     # dense type


# The plan takes the fused rotary product for every block format of q|k|v.
NORMED_ROPE = [(Q4_K, 32, 8, 128, 37), (Q4_K, 32, 8, 128, 0), (Q4_K, 32, 4, 64, 300), (Q4_K, 32, 8, 128, 512),
               (Q6_K, 32, 8, 128, 37), (Q8_0, 32, 8, 128, 200), (Q4_0, 32, 4, 64, 5)]


@pytest.mark.parametrize("t,heads,kv_heads,width,position", NORMED_ROPE,
                         ids=[f"{TYPE_NAMES[c[0]]}-{c[1]}/{c[2]}x{c[3]}-at{c[4]}" for c in NORMED_ROPE])
def test_matvec_normed_rope_equals_two_steps(env, t, heads, kv_heads, width, position):
    rt, L, stream = env
    kern = Kernels()
    cols, capacity = 4096, 512
    qd, kvd = heads * width, kv_heads * width
    rows = qd + 2 * kvd
    assert L.nya_hip_matvec_normed_rope(0, t, rows, cols, 0, 0, 0, 0, 1e-5, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0,
                                        stream) == 0
    rng = np.random.default_rng(rows + position)
    x = (3 * rng.standard_normal(cols)).astype(np.float32)
    r = rng.standard_normal(cols).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    cache_k = rng.standard_normal((capacity, kvd)).astype(np.float32)
    cache_v = rng.standard_normal((capacity, kvd)).astype(np.float32)
    freq = (10000.0 ** (-np.arange(width // 2) * 2.0 / width)).astype(np.float32)
    w = kern.device_weights(synth.weights(t, rows, cols, seed=rows), t, rows, cols)
    dev = Dev(rt)
    try:
        wd, xd, rd, gd = dev.put(w), dev.put(x), dev.put(r), dev.put(g)
        k1, v1, k2, v2 = dev.put(cache_k), dev.put(cache_v), dev.put(cache_k), dev.put(cache_v)
        fd, pd = dev.put(freq), dev.put(np.array([position], np.int32))
        h1, h2, y1, y2 = dev.empty(4 * cols), dev.empty(4 * cols), dev.empty(4 * rows), dev.empty(4 * rows)
        print(f"normed_rope {TYPE_NAMES[t]} {heads}/{kv_heads} width {width} position {position}", flush=True)
        assert L.nya_hip_matvec_normed_rope(wd, t, rows, cols, 0, xd, rd, gd, 1e-5, h1, y1, pd, fd, heads, kv_heads,
                                            width, capacity, k1, v1, stream) == 0
        assert L.nya_hip_matvec_normed(wd, t, rows, cols, xd, rd, gd, 1e-5, h2, y2, stream) == 0
        assert L.nya_hip_rope_qkv(y2, rows, y2 + 4 * qd, rows, y2 + 4 * (qd + kvd), rows, 1, heads, kv_heads, width,
                                  fd, pd, capacity, k2, v2, stream) == 0
        rt.sync(stream)
        bits = lambda p, like: dev.get(p, like).view(np.uint32)
        assert np.array_equal(bits(y1, np.empty(rows, np.float32)), bits(y2, np.empty(rows, np.float32)))
        assert np.array_equal(bits(k1, cache_k), bits(k2, cache_k))
        assert np.array_equal(bits(v1, cache_v), bits(v2, cache_v))
        assert np.array_equal(bits(h1, np.empty(cols, np.float32)), bits(h2, np.empty(cols, np.float32)))
    finally:
        dev.close()


ROPE_PARTS = [("qk|v", Q4_K, Q6_K, "qk"), ("q|kv", Q4_K, Q8_0, "q")]


@pytest.mark.parametrize("name,t0,t1,split", ROPE_PARTS, ids=[c[0] for c in ROPE_PARTS])
def test_matvec_rope_parts(env, oracle, name, t0, t1, split):
    """q|k|v rows stored as two matrices of different types (a Q4_K_M
    model's Q6_K value matrix): one normed rotary product per part, the
    first adding the residual, the second reading the updated residual,
    equal bit for bit the normed products of the parts followed by one
    rotary step over the rows put together; the scaled form per part is
    within the contract bounds of that (8B heads, position 77). Q4_K then
    Q6_K: both parts in one launch (nya_hip_matvec_rope_pair, normed and
    scaled forms) equal the per-part launches bit for bit."""
    rt, L, stream = env
    kern = Kernels()
    heads, kv_heads, width, cols, capacity, position = 32, 8, 128, 4096, 512, 77
    qd, kvd = heads * width, kv_heads * width
    rows = qd + 2 * kvd
    cut = qd + kvd if split == "qk" else qd
    shapes = [(t0, cut, 0), (t1, rows - cut, cut)]
    rng = np.random.default_rng(cut)
    x = (3 * rng.standard_normal(cols)).astype(np.float32)
    r = rng.standard_normal(cols).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    cache_k = rng.standard_normal((capacity, kvd)).astype(np.float32)
    cache_v = rng.standard_normal((capacity, kvd)).astype(np.float32)
    freq = (10000.0 ** (-np.arange(width // 2) * 2.0 / width)).astype(np.float32)
    host = [synth.weights(t, n, cols, seed=n + 3) for t, n, _ in shapes]
    dev = Dev(rt)
    try:
        wd = [dev.put(kern.device_weights(hw, t, n, cols)) for hw, (t, n, _) in zip(host, shapes)]
        xd, rd, gd = dev.put(x), dev.put(r), dev.put(g)
        k1, v1, k2, v2 = dev.put(cache_k), dev.put(cache_v), dev.put(cache_k), dev.put(cache_v)
        k3, v3 = dev.put(cache_k), dev.put(cache_v)
        fd, pd = dev.put(freq), dev.put(np.array([position], np.int32))
        h1, h2 = dev.empty(4 * cols), dev.empty(4 * cols)
        y1, y2, y3 = dev.empty(4 * rows), dev.empty(4 * rows), dev.empty(4 * rows)
        for (t, n, first), w in zip(shapes, wd):
            assert L.nya_hip_matvec_normed_rope(0, t, n, cols, 0, 0, 0, 0, 1e-5, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0,
                                                stream) == 0
        print(f"rope parts {name}", flush=True)
        # The parts: the first adds r into x (h to h1), the second reads h1.
        (t, n, first), w = shapes[0], wd[0]
        assert L.nya_hip_matvec_normed_rope(w, t, n, cols, first, xd, rd, gd, 1e-5, h1, y1, pd, fd, heads, kv_heads,
                                            width, capacity, k1, v1, stream) == 0
        (t, n, first), w = shapes[1], wd[1]
        assert L.nya_hip_matvec_normed_rope(w, t, n, cols, first, h1, 0, gd, 1e-5, 0, y1 + 4 * first, pd, fd, heads,
                                            kv_heads, width, capacity, k1, v1, stream) == 0
        # The separate steps.
        (t, n, first), w = shapes[0], wd[0]
        assert L.nya_hip_matvec_normed(w, t, n, cols, xd, rd, gd, 1e-5, h2, y2, stream) == 0
        (t, n, first), w = shapes[1], wd[1]
        assert L.nya_hip_matvec_normed(w, t, n, cols, h2, 0, gd, 1e-5, 0, y2 + 4 * first, stream) == 0
        assert L.nya_hip_rope_qkv(y2, rows, y2 + 4 * qd, rows, y2 + 4 * (qd + kvd), rows, 1, heads, kv_heads, width,
                                  fd, pd, capacity, k2, v2, stream) == 0
        # The scaled form of each part, from h * g and its partial sums.
        hv = (x + r).astype(np.float32)
        hd = hv.astype(np.float64)
        parts = np.zeros(NORM_PARTS)
        for j in range(0, cols, 16):
            parts[j // 16] = float((hd[j:j + 16] ** 2).sum())
        hnd, prd = dev.put(hv * g), dev.put(parts)
        for (t, n, first), w in zip(shapes, wd):
            assert L.nya_hip_matvec_scaled_rope(w, t, n, cols, first, hnd, prd, 1e-5, y3 + 4 * first, pd, fd, heads,
                                                kv_heads, width, capacity, k3, v3, stream) == 0
        pair = L.nya_hip_matvec_rope_pair(0, t0, cut, 0, t1, rows - cut, cols, 0, 0, 0, 0, 0, 1e-5, 0, 0, 0, 0, 0,
                                          0, 0, 0, 0, stream)
        assert pair == (0 if (t0, t1) == (Q4_K, Q6_K) else 1)
        if pair == 0:
            k4, v4, k5, v5 = dev.put(cache_k), dev.put(cache_v), dev.put(cache_k), dev.put(cache_v)
            h4, y4, y5 = dev.empty(4 * cols), dev.empty(4 * rows), dev.empty(4 * rows)
            assert L.nya_hip_matvec_rope_pair(wd[0], t0, cut, wd[1], t1, rows - cut, cols, xd, rd, gd, h4, 0, 1e-5,
                                              y4, pd, fd, heads, kv_heads, width, capacity, k4, v4, stream) == 0
            assert L.nya_hip_matvec_rope_pair(wd[0], t0, cut, wd[1], t1, rows - cut, cols, hnd, 0, 0, 0, prd, 1e-5,
                                              y5, pd, fd, heads, kv_heads, width, capacity, k5, v5, stream) == 0
        assert L.nya_hip_matvec_normed_rope(wd[1], t1, rows - cut, cols, cut + 1, xd, 0, gd, 1e-5, 0, y3, pd, fd,
                                            heads, kv_heads, width, capacity, k3, v3, stream) == 1   # odd first row
        assert L.nya_hip_matvec_normed_rope(wd[1], t1, rows - cut, cols, cut + 2, xd, 0, gd, 1e-5, 0, y3, pd, fd,
                                            heads, kv_heads, width, capacity, k3, v3, stream) == 1   # past the rows
        rt.sync(stream)
        bits = lambda p, like: dev.get(p, like).view(np.uint32)
        assert np.array_equal(bits(y1, np.empty(rows, np.float32)), bits(y2, np.empty(rows, np.float32)))
        assert np.array_equal(bits(k1, cache_k), bits(k2, cache_k))
        assert np.array_equal(bits(v1, cache_v), bits(v2, cache_v))
        assert np.array_equal(bits(h1, np.empty(cols, np.float32)), bits(h2, np.empty(cols, np.float32)))
        if pair == 0:
            for got, want, like in ((y4, y1, np.empty(rows, np.float32)), (k4, k1, cache_k), (v4, v1, cache_v),
                                    (h4, h1, np.empty(cols, np.float32)), (y5, y3, np.empty(rows, np.float32)),
                                    (k5, k3, cache_k), (v5, v3, cache_v)):
                assert np.array_equal(bits(got, like), bits(want, like))
        a = dev.get(y3, np.empty(rows, np.float32))
        b = dev.get(y2, np.empty(rows, np.float32))
        ka, kb = dev.get(k3, cache_k), dev.get(k2, cache_k)
        va, vb = dev.get(v3, cache_v), dev.get(v2, cache_v)
    finally:
        dev.close()
    xnd = hd / np.sqrt(np.mean(hd * hd) + 1e-5) * g.astype(np.float64)
    mags = np.concatenate([oracle.contract_sums(hw, t, xnd, n, cols)[1][0] for hw, (t, n, _) in zip(host, shapes)])
    m = 2e-6 * (1 + mags)
    bound = m + m[np.arange(rows) ^ 1]
    for got, want, bd, what in ((a, b, bound, "rows"), (ka[position], kb[position], bound[qd:qd + kvd], "key"),
                                (va[position], vb[position], bound[qd + kvd:], "value")):
        err = np.abs(got.astype(np.float64) - want) / (bd + 1e-6 * np.abs(want))
        assert err.max() <= 1, f"scaled parts, {what}: worst {err.max():.3g}"


@pytest.mark.parametrize("t,heads,kv_heads,width,position", NORMED_ROPE,
                         ids=[f"{TYPE_NAMES[c[0]]}-{c[1]}/{c[2]}x{c[3]}-at{c[4]}" for c in NORMED_ROPE])
def test_matvec_scaled_rope(env, oracle, t, heads, kv_heads, width, position):
    """The rotary q|k|v product of hn = h * g with the norm's scale from
    partial sums of squares, against nya_hip_matvec_normed_rope of h (bit for
    bit the norm step, the product and the rotary step): the two differ only
    in the row sums, each within the contract bound 1e-6 (1 + sum |w xn|)
    (backend/tests/test_quant_kernels.c:13-25), so every output (a row sum,
    or a rotation c a -/+ s b of a pair of them) is within twice the bounds
    of its rows plus 1e-6 of its value; the cache slot of the position gets
    the same rows within the same bound and every other slot is untouched
    (at position 512 = capacity: nothing rotated or stored)."""
    rt, L, stream = env
    kern = Kernels()
    cols, capacity = 4096, 512
    qd, kvd = heads * width, kv_heads * width
    rows = qd + 2 * kvd
    assert L.nya_hip_matvec_scaled_rope(0, t, rows, cols, 0, 0, 0, 1e-5, 0, 0, 0, 0, 0, 0, 0, 0, 0, stream) == 0
    rng = np.random.default_rng(rows + position + 5)
    h = (3 * rng.standard_normal(cols)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    hd = h.astype(np.float64)
    parts = np.zeros(NORM_PARTS)
    for j in range(0, cols, 16):
        parts[j // 16] = float((hd[j:j + 16] ** 2).sum())
    cache_k = rng.standard_normal((capacity, kvd)).astype(np.float32)
    cache_v = rng.standard_normal((capacity, kvd)).astype(np.float32)
    freq = (10000.0 ** (-np.arange(width // 2) * 2.0 / width)).astype(np.float32)
    host = synth.weights(t, rows, cols, seed=rows)
    w = kern.device_weights(host, t, rows, cols)
    dev = Dev(rt)
    try:
        wd, xd, gd, hnd, prd = dev.put(w), dev.put(h), dev.put(g), dev.put(h * g), dev.put(parts)
        k1, v1, k2, v2 = dev.put(cache_k), dev.put(cache_v), dev.put(cache_k), dev.put(cache_v)
        fd, pd = dev.put(freq), dev.put(np.array([position], np.int32))
        y1, y2 = dev.empty(4 * rows), dev.empty(4 * rows)
        print(f"scaled_rope {TYPE_NAMES[t]} {heads}/{kv_heads} width {width} position {position}", flush=True)
        assert L.nya_hip_matvec_scaled_rope(wd, t, rows, cols, 0, hnd, prd, 1e-5, y1, pd, fd, heads, kv_heads, width,
                                            capacity, k1, v1, stream) == 0
        assert L.nya_hip_matvec_normed_rope(wd, t, rows, cols, 0, xd, 0, gd, 1e-5, 0, y2, pd, fd, heads, kv_heads,
                                            width, capacity, k2, v2, stream) == 0
        rt.sync(stream)
        got = lambda p, like: dev.get(p, np.empty_like(like))
        a, b = got(y1, np.empty(rows, np.float32)), got(y2, np.empty(rows, np.float32))
        ka, kb, va, vb = got(k1, cache_k), got(k2, cache_k), got(v1, cache_v), got(v2, cache_v)
    finally:
        dev.close()
    xnd = hd / np.sqrt(np.mean(hd * hd) + 1e-5) * g.astype(np.float64)
    _, mags = oracle.contract_sums(host, t, xnd, rows, cols)
    m = 2e-6 * (1 + mags[0])
    bound = m + m[np.arange(rows) ^ 1]
    check = lambda x, y, bd, what: np.all(np.abs(x.astype(np.float64) - y) <= bd + 1e-6 * np.abs(y)) or \
        pytest.fail(f"{what}: worst {float((np.abs(x.astype(np.float64) - y) / (bd + 1e-6 * np.abs(y))).max()):.3g}")
    check(a, b, bound, "q|k|v rows")
    others = np.arange(capacity) != position
    assert np.array_equal(ka[others], cache_k[others]) and np.array_equal(va[others], cache_v[others])
    if position < capacity:
        check(ka[position], kb[position], bound[qd:qd + kvd], "cached key")
        check(va[position], vb[position], bound[qd + kvd:], "cached value")
    else:
        assert np.array_equal(ka, cache_k) and np.array_equal(va, cache_v)

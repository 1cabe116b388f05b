"""TEST INFRASTRUCTURE ONLY: the engine's sampler and its speculative
sampling loop, restated in Python as the oracle of
nya_compute_generate_sampled. Only tests/ use it; the product never does.

Each function follows the reference lines it names, with the same float /
double arithmetic: float32 logits and probabilities, double masses and
CDFs, the C library's expf (called through ctypes, so the exponentials are
the ones the C code gets), and the engine's random stream.

The loop takes its logits from two callables, so the same rule runs on any
source of logits: the engine's own scalar sessions (which pins this
restatement to the engine's nya_llm_generate_draft token for token,
tests/test_sampling_oracle.py) or a provider's plans (the oracle of the
batched implementation).

Pinning (tests/test_sampling_oracle.py):
 - Stream, distribution, sample, draw and generate: token for token equal to
   the engine's nya_llm_generate_draft and nya_llm_generate compiled from
   the reference sources (oracle/_ref/libnya_dropin.so), over seeds,
   temperatures, top-k, top-p, windows and drafts.
The engine's own distribution checks (backend/tests/test_generation.c
:345-387: the first token's frequency over many seeds, top-p keeping only
the leading candidate) run on the batched implementation
(tests/test_speculative.py).
"""
from __future__ import annotations

import ctypes
import ctypes.util
import math
from typing import Callable, Sequence

import numpy as np

_libm = ctypes.CDLL(ctypes.util.find_library("m") or "libm.so.6")
_libm.expf.restype = ctypes.c_float
_libm.expf.argtypes = [ctypes.c_float]

MASK64 = (1 << 64) - 1
DEFAULT_SEED = 0x9E3779B97F4A7C15   # backend/core/llm_cpu.c:1229
DRAFT_STREAM = 0xD1B54A32D192ED03   # llm_cpu.c:1230


def f32(v) -> float:
    return float(np.float32(v))


class Stream:
    """The engine's random stream (backend/core/llm_cpu.c:798-808)."""

    def __init__(self, state: int):
        self.state = state & MASK64

    def u32(self) -> int:
        s = self.state
        s ^= s >> 12
        s = (s ^ (s << 25)) & MASK64
        s ^= s >> 27
        self.state = s
        return ((s * 0x2545F4914F6CDD1D) & MASK64) >> 32

    def unit(self) -> float:
        # (float)(u32 >> 8) / 16777216.0f: exact, k / 2^24.
        return (self.u32() >> 8) / 16777216.0


def distribution(logits: np.ndarray, temperature: float, top_p: float, top_k: int):
    """llm_cpu.c:847-888: (dense probabilities, [(token, probability)] in
    candidate order), or None where the engine returns -1."""
    logits = np.asarray(logits, dtype=np.float32)
    n = logits.size
    kept = n if top_k == 0 or top_k > n else top_k
    if n == 0 or not temperature > 0.0:
        return None
    if np.isnan(logits).any() or (logits == np.inf).any():
        return None
    # Larger value first, then smaller token (llm_cpu.c:811-826).
    order = sorted(range(n), key=lambda t: (-float(logits[t]), t))[:kept]
    top = float(logits[order[0]])
    if not math.isfinite(top):
        return None
    t32 = np.float32(temperature)
    values = []
    mass = 0.0
    for t in order:
        arg = np.float32(np.float32(logits[t]) - np.float32(top)) / t32
        e = float(_libm.expf(float(np.float32(arg))))
        values.append(e)
        mass += e
    prefix = 0.0
    cut = float(np.float32(top_p)) * mass
    for j, e in enumerate(values):
        prefix += e
        if prefix >= cut:
            kept = j + 1
            break
    if not prefix > 0.0 or not math.isfinite(prefix):
        return None
    dense = np.zeros(n, dtype=np.float32)
    cand = []
    for j in range(kept):
        p = f32(values[j] / prefix)
        dense[order[j]] = p
        cand.append((order[j], p))
    return dense, cand


def sample(logits: np.ndarray, temperature: float, top_p: float, top_k: int, rng: Stream):
    """llm_cpu.c:890-911: (token, dense distribution or None at temperature 0)."""
    logits = np.asarray(logits, dtype=np.float32)
    if temperature == 0.0:
        if np.isnan(logits).any() or (logits == np.inf).any():
            return None
        best = int(np.argmax(logits))   # the first largest
        if not math.isfinite(float(logits[best])):
            return None
        return best, None
    d = distribution(logits, temperature, top_p, top_k)
    if d is None:
        return None
    dense, cand = d
    target = rng.unit()
    cdf = 0.0
    for token, p in cand:
        cdf += p
        if target < cdf:
            return token, dense
    return cand[-1][0], dense


def draw(weights: np.ndarray, rng: Stream):
    """llm_cpu.c:915-932: one token from a dense nonnegative float vector."""
    w = np.asarray(weights, dtype=np.float32)
    if (w < 0).any() or not np.isfinite(w).all():
        return None
    mass = 0.0
    for v in w:
        mass += float(v)
    positive = np.nonzero(w > 0)[0]
    if not mass > 0.0:
        return None
    last = int(positive[-1])
    target = rng.unit() * mass
    cdf = 0.0
    for j, v in enumerate(w):
        cdf += float(v)
        if target < cdf:
            return j
    return last


# target_rows(prefix, tokens) -> rows: rows[j] are the target's logits after
#   prefix + tokens[0..j] (tokens[0] at position len(prefix)).
# draft_row(prefix, token) -> the draft's logits after prefix + [token].
RowsFn = Callable[[Sequence[int], Sequence[int]], np.ndarray]
RowFn = Callable[[Sequence[int], int], np.ndarray]


def generate(target_rows: RowsFn, draft_row: RowFn | None, prompt: Sequence[int], limit: int, window: int,
             temperature: float, top_p: float = 1.0, top_k: int = 0, seed: int = 0, stops=()):
    """The engine's speculative sampling loop for an ordinary draft
    (llm_cpu.c:1215-1317), or its plain loop without one (:1036-1075):
    (tokens, {"accepted": .., "draft_tokens": ..}). The draft runs each
    proposal before sampling the next (its logits after pending, p_0, ..);
    the target's rows of a round are requested in one call."""
    rng = Stream(seed if seed else DEFAULT_SEED)
    draft_rng = Stream(rng.state ^ DRAFT_STREAM)
    if draft_rng.state == 0:
        draft_rng.state = 1
    if draft_row is None:
        window = 0
    stops = set(stops)
    out: list[int] = []
    seq = list(prompt)
    P = len(prompt) - 1
    accepted_total = drafted = 0
    stopped = False
    while not stopped and len(out) < limit:
        m = min(window, limit - len(out))
        batch = [seq[P]]
        qs = []
        for i in range(m):
            row = draft_row(seq[:P] + batch[:i], batch[i])
            r = sample(row, temperature, top_p, top_k, draft_rng)
            assert r is not None, "draft sampling failed"
            token, q = r
            qs.append(q)
            batch.append(token)
            drafted += 1
            if token in stops:
                m = i + 1
                break
        rows = target_rows(seq[:P], batch[:m + 1])
        emitted = 0
        rejected = False
        for j in range(m):
            if stopped:
                break
            token = batch[j + 1]
            q = qs[j]
            d = distribution(rows[j], temperature, top_p, top_k)
            assert d is not None, "target distribution failed"
            p = d[0]
            assert q[token] > 0
            accepted = rng.unit() * float(q[token]) < float(p[token])
            if not accepted:
                residual = np.maximum(p - q, np.float32(0)).astype(np.float32)
                token = draw(residual, rng)
                assert token is not None
            else:
                accepted_total += 1
            out.append(token)
            seq.append(token)
            emitted += 1
            if token in stops:
                stopped = True
            if not accepted:
                rejected = True
                break
        if not rejected and not stopped and len(out) < limit:
            r = sample(rows[m], temperature, top_p, top_k, rng)
            assert r is not None, "target sampling failed"
            token = r[0]
            out.append(token)
            seq.append(token)
            emitted += 1
            if token in stops:
                stopped = True
        P += emitted
    return out, {"accepted": accepted_total, "draft_tokens": drafted}

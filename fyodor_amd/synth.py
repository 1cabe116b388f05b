"""Seeded synthetic GGUF matrices and activations for the benchmark and tests.

Value distributions are the ones the benchmark workloads name:
  Q8_0  q uniform in [-127, 127], d = f16(|N(0, 0.02)| / 127)
  Q4_0  q uniform in [0, 15] (random bytes), d = f16(|N(0, 0.02)| / 8)
  Q4_K  scales[12] and qs[128] uniform random bytes (every pattern is valid),
        d = f16(|N(0, 0.02)| / 945), dmin = f16(|N(0, 0.02)| / 63)
  Q6_K  ql, qh uniform bytes, sc uniform int8, d = f16(|N(0, 0.02)| / 4096)
  x     fp32 N(0, 1)
f16 values are rounded to nearest even (numpy's float32 -> float16), as the
reference encoder does (backend/core/llm_quant.c:46-67). Everything derives
from one numpy PCG64 stream per seed, so the same seed gives the same bytes.
"""
from __future__ import annotations

import hashlib

import numpy as np

from . import BF16, F16, F32, Q4_0, Q4_K, Q6_K, Q8_0, storage_bytes


def _scales(rng: np.random.Generator, n: int, divisor: float) -> np.ndarray:
    v = np.abs(rng.normal(0.0, 0.02, n)).astype(np.float32) / np.float32(divisor)
    return v.astype(np.float16).view(np.uint16)


def weights(type_id: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """GGUF bytes of a [rows, cols] matrix as a flat uint8 array."""
    rng = np.random.default_rng(seed)
    nbytes = storage_bytes(type_id, rows, cols)
    if type_id == F32:
        return rng.standard_normal(rows * cols, dtype=np.float32).view(np.uint8).copy()
    if type_id in (F16, BF16):
        v = rng.standard_normal(rows * cols, dtype=np.float32)
        if type_id == F16:
            return v.astype(np.float16).view(np.uint8).copy()
        bits = v.view(np.uint32)
        return ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16).view(np.uint8).copy()
    raw = np.frombuffer(rng.bytes(nbytes), dtype=np.uint8).copy()
    if type_id == Q8_0:
        blk = raw.reshape(-1, 34)
        n = blk.shape[0]
        blk[:, 0:2] = _scales(rng, n, 127.0).view(np.uint8).reshape(n, 2)
        q = rng.integers(-127, 128, size=(n, 32), dtype=np.int16).astype(np.int8)
        blk[:, 2:] = q.view(np.uint8)
    elif type_id == Q4_0:
        blk = raw.reshape(-1, 18)
        n = blk.shape[0]
        blk[:, 0:2] = _scales(rng, n, 8.0).view(np.uint8).reshape(n, 2)
    elif type_id == Q4_K:
        blk = raw.reshape(-1, 144)
        n = blk.shape[0]
        blk[:, 0:2] = _scales(rng, n, 945.0).view(np.uint8).reshape(n, 2)
        blk[:, 2:4] = _scales(rng, n, 63.0).view(np.uint8).reshape(n, 2)
    elif type_id == Q6_K:
        blk = raw.reshape(-1, 210)
        n = blk.shape[0]
        blk[:, 208:210] = _scales(rng, n, 32.0 * 128.0).view(np.uint8).reshape(n, 2)
    else:
        raise ValueError(f"unsupported type {type_id}")
    return raw


def activations(batch: int, cols: int, seed: int) -> np.ndarray:
    """X [batch, cols] fp32 ~ N(0, 1)."""
    rng = np.random.default_rng(seed ^ 0x5A5A5A5A)
    return rng.standard_normal((batch, cols), dtype=np.float32)


def digest(*arrays: np.ndarray) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).view(np.uint8).tobytes())
    return h.hexdigest()[:16]

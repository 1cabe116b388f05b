"""Deterministic inputs restated from the reference's own tests.

- pattern_matrix / pass_input / batch_inputs: backend/tests/test_quant_kernels.c
  :154-175 and :191 (byte pattern (i*73 + i/17 + 31) & 255 with fixed scale
  bytes, x = ((i + 3*pass) % 97 - 48) / 49, batch inputs (i % 61 - 30) / 31);
- k_quant_fixture: backend/tests/test_architectures.c:229-300, Q4_K/Q6_K
  blocks built from logical scales and integers by an encoder that is
  independent of any decoder, with their exact element values;
- constant_rows: backend/tests/test_generation.c:79-103, Q4_0/Q8_0 rows with
  power-of-two scales whose products are exact.
"""
import numpy as np

from fyodor_amd import BF16, F16, F32, Q4_0, Q4_K, Q6_K, Q8_0, storage_bytes


def pattern_matrix(type_id: int, rows: int, cols: int) -> np.ndarray:
    n = storage_bytes(type_id, rows, cols)
    i = np.arange(n, dtype=np.int64)
    data = ((i * 73 + i // 17 + 31) & 255).astype(np.uint8)
    if type_id in (F32, F16, BF16):
        k = np.arange(rows * cols, dtype=np.int64)
        value = ((k % 127) - 63).astype(np.float32) / np.float32(64)
        if type_id == F32:
            return value.view(np.uint8).copy()
        if type_id == BF16:
            return (value.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).copy()
        v = (0x3000 + (k % 1024) + np.where(k % 2 == 1, 0x8000, 0)).astype(np.uint16)
        return v.view(np.uint8).copy()
    block = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q6_K: 210}[type_id]
    scale = 208 if type_id == Q6_K else 0
    starts = np.arange(0, n, block)
    data[starts + scale] = 0
    data[starts + scale + 1] = 0x28
    if type_id == Q4_K:
        data[starts + 2] = 0
        data[starts + 3] = 0x24
    return data


def pass_input(cols: int, p: int) -> np.ndarray:
    i = np.arange(cols)
    return (((i + p * 3) % 97) - 48).astype(np.float32) / np.float32(49)


def batch_inputs(batch: int, cols: int) -> np.ndarray:
    i = np.arange(batch * cols)
    return (((i % 61) - 30).astype(np.float32) / np.float32(31)).reshape(batch, cols)


def k_quant_fixture(kind: str):
    """(bytes of 2 rows x 512 columns, exact element values, x) for Q4_K or Q6_K."""
    x = ((np.arange(512) % 23) - 11).astype(np.float32) / np.float32(16)
    expected = np.zeros(1024, dtype=np.float32)
    if kind == "Q4_K":
        data = np.zeros(4 * 144, dtype=np.uint8)
        for b in range(4):
            p = data[b * 144:(b + 1) * 144]
            p[1], p[3] = 0x38, 0x34                 # d = 1/2, dmin = 1/4
            sc = [(g * 11 + b * 7) % 64 for g in range(8)]
            mn = [(g * 17 + b * 13) % 64 for g in range(8)]
            for g in range(4):
                p[4 + g] = sc[g] | ((sc[g + 4] >> 4) << 6)
                p[8 + g] = mn[g] | ((mn[g + 4] >> 4) << 6)
                p[12 + g] = (sc[g + 4] & 15) | ((mn[g + 4] & 15) << 4)
            for pair in range(4):
                for j in range(32):
                    lo = (j * 3 + pair + b) % 16
                    hi = (j * 7 + pair * 3 + b) % 16
                    p[16 + pair * 32 + j] = lo | (hi << 4)
                    expected[b * 256 + pair * 64 + j] = 0.5 * sc[pair * 2] * lo - 0.25 * mn[pair * 2]
                    expected[b * 256 + pair * 64 + 32 + j] = 0.5 * sc[pair * 2 + 1] * hi - 0.25 * mn[pair * 2 + 1]
        return data, expected, x
    data = np.zeros(4 * 210, dtype=np.uint8)
    for b in range(4):
        p = data[b * 210:(b + 1) * 210]
        p[209] = 0x30                               # d = 1/8
        sc = [((g * 37 + b * 53) % 256) - 128 for g in range(16)]
        for g in range(16):
            p[192 + g] = sc[g] & 255
        for half in range(2):
            for j in range(32):
                q = [(j * 13 + k * 19 + half * 31 + b * 7) % 64 for k in range(4)]
                for k in range(4):
                    n = half * 128 + k * 32 + j
                    expected[b * 256 + n] = 0.125 * sc[n // 16] * (q[k] - 32)
                p[half * 64 + j] = (q[0] & 15) | ((q[2] & 15) << 4)
                p[half * 64 + 32 + j] = (q[1] & 15) | ((q[3] & 15) << 4)
                p[128 + half * 32 + j] = (q[0] >> 4) | ((q[1] >> 4) << 2) | ((q[2] >> 4) << 4) | ((q[3] >> 4) << 6)
    return data, expected, x


def constant_rows(type_id: int, rows: int, cols: int, value: float) -> np.ndarray:
    """Every weight equal to `value` (1, 1/32 or 1/64) in Q4_0 or Q8_0."""
    half = {1.0: 0x3C00, 0.03125: 0x2800, 0.015625: 0x2400}[value]
    block = [half & 255, half >> 8] + ([0x99] * 16 if type_id == Q4_0 else [1] * 32)
    return np.tile(np.array(block, dtype=np.uint8), rows * cols // 32)

"""Result checks shared by the GPU parity tests.

check_rows restates the reference kernel contract's bound
(backend/tests/test_quant_kernels.c:138-213): every output row within
1e-6 * (1 + sum |w x|) of the double-precision dot, and optionally the first
rows within 1.5e-4 * (1 + |y|) of the scalar kernel.
"""
import numpy as np

from fyodor_amd import TYPE_NAMES


def check_rows(oracle, w, t, x, rows, cols, actual, scalar=None, first_rows=0):
    s, m = oracle.matvec_double(w, t, x, rows, cols)
    err = np.abs(actual.astype(np.float64) - s)
    bad = ~np.isfinite(actual) | (err > 1e-6 * (1 + m))
    assert not bad.any(), f"{TYPE_NAMES[t]} rows {np.nonzero(bad)[0][:5]}: {actual[bad][:3]} vs {s[bad][:3]}"
    if scalar is not None and first_rows:
        a, e = actual[:first_rows], scalar[:first_rows]
        assert np.all(np.abs(a - e) <= np.float32(0.00015) * (1 + np.abs(e)))


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))

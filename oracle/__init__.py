"""TEST INFRASTRUCTURE ONLY: ctypes access to the parity oracle.

``liboracle.so`` is this repository's C restatement of the reference scalar
path (quant_oracle.c). ``_ref/libnya_ref.so`` is the reference's own CPU path
compiled from its sources by ``make -C oracle ref`` where they are mounted.
Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use
this package; the product never does.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIBRARY = HERE / "liboracle.so"
REFERENCE_LIBRARY = HERE / "_ref" / "libnya_ref.so"

_F = ctypes.POINTER(ctypes.c_float)
_D = ctypes.POINTER(ctypes.c_double)
_B = ctypes.c_void_p
_S = ctypes.c_size_t


def _fp(a):
    return a.ctypes.data_as(_F)


def _dp(a):
    return a.ctypes.data_as(_D)


class Oracle:
    """The C restatement (quant_oracle.c)."""

    def __init__(self):
        if not ORACLE_LIBRARY.exists():
            subprocess.run(["make", "-C", str(HERE), "oracle"], check=True, capture_output=True)
        lib = ctypes.CDLL(str(ORACLE_LIBRARY))
        lib.orc_half.restype = ctypes.c_float
        lib.orc_half.argtypes = [_B]
        lib.orc_round_f16.restype = ctypes.c_float
        lib.orc_round_f16.argtypes = [ctypes.c_float]
        lib.orc_value.restype = ctypes.c_float
        lib.orc_value.argtypes = [_B, ctypes.c_uint, _S]
        lib.orc_matvec.argtypes = [_F, _B, ctypes.c_uint, _F, _S, _S]
        lib.orc_matvec_double.argtypes = [_D, _D, _B, ctypes.c_uint, _F, _S, _S]
        lib.orc_matmul.argtypes = [_F, _B, ctypes.c_uint, _F, _S, _S, _S, ctypes.c_int]
        lib.orc_dequant.argtypes = [_F, _B, ctypes.c_uint, _S, _S, ctypes.c_int]
        self.lib = lib

    def half(self, bits: int) -> float:
        b = np.array([bits & 255, bits >> 8], dtype=np.uint8)
        return self.lib.orc_half(b.ctypes.data)

    def round_f16(self, v: float) -> float:
        return self.lib.orc_round_f16(v)

    def values(self, w: np.ndarray, type_id: int, count: int) -> np.ndarray:
        return np.array([self.lib.orc_value(w.ctypes.data, type_id, i) for i in range(count)], dtype=np.float32)

    def matvec(self, w: np.ndarray, type_id: int, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(rows, dtype=np.float32)
        self.lib.orc_matvec(_fp(y), w.ctypes.data, type_id, _fp(x), cols, rows)
        return y

    def matvec_double(self, w: np.ndarray, type_id: int, x: np.ndarray, rows: int, cols: int):
        x = np.ascontiguousarray(x, dtype=np.float32)
        s = np.empty(rows, dtype=np.float64)
        m = np.empty(rows, dtype=np.float64)
        self.lib.orc_matvec_double(_dp(s), _dp(m), w.ctypes.data, type_id, _fp(x), cols, rows)
        return s, m

    def matmul(self, w: np.ndarray, type_id: int, x: np.ndarray, rows: int, cols: int, batch: int,
               threads: int = 1) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(batch * rows, dtype=np.float32)
        self.lib.orc_matmul(_fp(y), w.ctypes.data, type_id, _fp(x), cols, rows, batch, threads)
        return y.reshape(batch, rows)

    def dequant(self, w: np.ndarray, type_id: int, rows: int, cols: int, threads: int = 0) -> np.ndarray:
        """[rows, cols] float32: every weight as the reference decodes it."""
        out = np.empty((rows, cols), dtype=np.float32)
        self.lib.orc_dequant(_fp(out), w.ctypes.data, type_id, rows, cols, threads or host_threads())
        return out

    def contract_sums(self, w: np.ndarray, type_id: int, x: np.ndarray, rows: int, cols: int):
        """Per token and row, the double sum of decoded products and the sum
        of their magnitudes (backend/tests/test_quant_kernels.c:13-25) for a
        whole batch X [batch, cols]: [batch, rows] each, from the decoded
        weights by float64 matrix products."""
        wd = self.dequant(w, type_id, rows, cols).astype(np.float64)
        xd = np.asarray(x, dtype=np.float64).reshape(-1, cols)
        s = xd @ wd.T
        np.abs(wd, out=wd)
        m = np.abs(xd) @ wd.T
        return s, m


def host_threads() -> int:
    """Threads for the oracle's threaded helpers: the CPUs this process may
    run on, at most 16."""
    import os
    try:
        return max(1, min(16, len(os.sched_getaffinity(0))))
    except (AttributeError, OSError):
        return max(1, min(16, os.cpu_count() or 1))


class Reference:
    """The reference CPU path built from its own sources (None if absent)."""

    def __init__(self):
        lib = ctypes.CDLL(str(REFERENCE_LIBRARY))
        lib.nya_llm_round_f16.restype = ctypes.c_float
        lib.nya_llm_round_f16.argtypes = [ctypes.c_float]
        lib.nya_llm_matvec.argtypes = [_B, _F, _B, _F, _S, _S]
        lib.nya_llm_tensor_value.restype = ctypes.c_float
        lib.nya_llm_tensor_value.argtypes = [_B, _S]
        lib.nya_compute_create_for.restype = _B
        lib.nya_compute_create_for.argtypes = [ctypes.c_char_p]
        lib.nya_compute_free.argtypes = [_B]
        lib.nya_compute_matmul_typed.argtypes = [_B, _B, _S, _S, ctypes.c_uint, _F, _F, _S]
        self.lib = lib

    @staticmethod
    def available() -> bool:
        return REFERENCE_LIBRARY.exists()

    def _tensor(self, w: np.ndarray, type_id: int):
        # nya_llm_tensor (backend/core/llm_internal.h:22-31): name[128], type,
        # dimension_count, dimensions[4], relative_offset, data, data_size, bound.
        class Tensor(ctypes.Structure):
            _fields_ = [("name", ctypes.c_char * 128), ("type", ctypes.c_uint32),
                        ("dimension_count", ctypes.c_uint32), ("dimensions", ctypes.c_uint64 * 4),
                        ("relative_offset", ctypes.c_uint64), ("data", ctypes.c_void_p),
                        ("data_size", ctypes.c_size_t), ("bound", ctypes.c_int)]
        t = Tensor()
        t.type = type_id
        t.data = w.ctypes.data
        t.data_size = w.nbytes
        return t

    def matvec(self, w: np.ndarray, type_id: int, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
        """The reference scalar kernel: nya_llm_matvec with no compute context."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(rows, dtype=np.float32)
        t = self._tensor(w, type_id)
        self.lib.nya_llm_matvec(None, _fp(y), ctypes.addressof(t), _fp(x), cols, rows)
        return y

    def value(self, w: np.ndarray, type_id: int, index: int) -> float:
        t = self._tensor(w, type_id)
        return self.lib.nya_llm_tensor_value(ctypes.addressof(t), index)

    def cpu_provider(self):
        """The reference CPU provider (threaded SIMD, backend/core/cpu_backend.c)."""
        ctx = self.lib.nya_compute_create_for(b"cpu")
        if not ctx:
            raise RuntimeError("reference CPU provider could not be created")
        return ctx

    def provider_matmul(self, ctx, w: np.ndarray, type_id: int, x: np.ndarray, rows: int, cols: int,
                        batch: int, out: np.ndarray) -> None:
        status = self.lib.nya_compute_matmul_typed(ctx, w.ctypes.data, rows, cols, type_id,
                                                   _fp(x), _fp(out), batch)
        if status != 0:
            raise RuntimeError("reference CPU provider declined")

    def free(self, ctx) -> None:
        self.lib.nya_compute_free(ctx)

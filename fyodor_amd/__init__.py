"""Python handle on the ROCm quantized-matrix provider.

The product is native: ``lib/libfyodor_rocm.so`` (the C provider behind the
engine's compute API, ``include/compute.h``) and ``lib/libfyodor_hip.so``
(the gfx950 kernels behind ``include/fyodor_hip.h``). This module only loads
them with ctypes so tests and the benchmark call the same C entry points the
engine calls (``nya_compute_matvec_typed`` / ``nya_compute_matmul_typed``,
backend/include/compute.h:78-83).

Unlike the engine, which silently recomputes on its CPU kernels when the
provider returns -1 (backend/core/llm_quant.c:159-160), this wrapper raises:
a declined or failed call is an error here, never a fallback.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

LIB_DIR = Path(__file__).resolve().parent / "lib"
PROVIDER_LIBRARY = LIB_DIR / "libfyodor_rocm.so"
KERNEL_LIBRARY = LIB_DIR / "libfyodor_hip.so"

# GGML storage type IDs (backend/core/llm_internal.h:11-19).
F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 2, 8, 12, 14, 30
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K", BF16: "BF16"}
# (elements per block, bytes per block) of GGUF storage.
BLOCKS = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}

CAP_MATVEC, CAP_QUANTIZED, CAP_RESIDENT, CAP_MATMUL = 1, 2, 4, 8


def storage_bytes(type_id: int, rows: int, cols: int) -> int:
    block, size = BLOCKS[type_id]
    assert cols % block == 0
    return rows * (cols // block) * size


class ComputeStats(ctypes.Structure):
    """nya_compute_stats (backend/include/compute.h:13-22)."""
    _fields_ = [
        ("weights_bytes", ctypes.c_size_t), ("kv_bytes", ctypes.c_size_t),
        ("scratch_bytes", ctypes.c_size_t), ("prefill_batch", ctypes.c_size_t),
        ("external_matmul_bytes", ctypes.c_size_t),
        ("kernel_launches", ctypes.c_ulonglong), ("uploads", ctypes.c_ulonglong),
        ("downloads", ctypes.c_ulonglong), ("synchronizations", ctypes.c_ulonglong),
        ("external_matmul_calls", ctypes.c_ulonglong),
        ("graph_captures", ctypes.c_ulonglong), ("graph_replays", ctypes.c_ulonglong),
        ("external_matmul_kind", ctypes.c_uint),
        ("cutlass_matmul_calls", ctypes.c_ulonglong), ("tiled_attention_calls", ctypes.c_ulonglong),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


class ProviderUnavailable(RuntimeError):
    pass


class ComputeDeclined(RuntimeError):
    pass


_provider = None


def compute_api(lib: ctypes.CDLL) -> ctypes.CDLL:
    """Declares the engine's compute API (include/compute.h) on a loaded
    library that exports it: this repository's provider library, or a
    build of the engine's own dispatcher with this provider registered."""
    vp, sz, fp = ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_float)
    lib.nya_compute_create_for.restype = vp
    lib.nya_compute_create_for.argtypes = [ctypes.c_char_p]
    lib.nya_compute_free.argtypes = [vp]
    lib.nya_compute_name.restype = ctypes.c_char_p
    lib.nya_compute_name.argtypes = [vp]
    lib.nya_compute_capabilities.restype = ctypes.c_uint
    lib.nya_compute_capabilities.argtypes = [vp]
    lib.nya_compute_matvec.argtypes = [vp, vp, sz, sz, fp, fp]
    lib.nya_compute_matvec_typed.argtypes = [vp, vp, sz, sz, ctypes.c_uint, fp, fp]
    lib.nya_compute_matmul_typed.argtypes = [vp, vp, sz, sz, ctypes.c_uint, fp, fp, sz]
    lib.nya_compute_context_stats.argtypes = [vp, ctypes.POINTER(ComputeStats)]
    lib.nya_compute_backend_known.argtypes = [ctypes.c_char_p]
    lib.nya_compute_backend_compiled.argtypes = [ctypes.c_char_p]
    return lib


def provider_library() -> ctypes.CDLL:
    """Loads libfyodor_rocm.so; raises when it has not been built."""
    global _provider
    if _provider is None:
        if not PROVIDER_LIBRARY.exists():
            raise ProviderUnavailable(f"{PROVIDER_LIBRARY} is missing: run `python -m fyodor_amd.build`")
        _provider = compute_api(ctypes.CDLL(str(PROVIDER_LIBRARY)))
    return _provider


def _float_ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


class Compute:
    """One nya_compute_context on the ROCm provider.

    Weight arrays passed in are kept referenced for the context's lifetime:
    the provider caches them by address (backend/include/compute.h:68-71).
    """

    def __init__(self, provider: str = "rocm"):
        if provider == "rocm" and "NYA_ROCM_KERNEL_LIBRARY" not in os.environ:
            if not KERNEL_LIBRARY.exists():
                raise ProviderUnavailable(f"{KERNEL_LIBRARY} is missing: run `python -m fyodor_amd.build`")
            os.environ["NYA_ROCM_KERNEL_LIBRARY"] = str(KERNEL_LIBRARY)
        self._lib = provider_library()
        self._ctx = self._lib.nya_compute_create_for(provider.encode())
        if not self._ctx:
            raise ProviderUnavailable(f"provider {provider!r} could not be created (see stderr)")
        self._borrowed = []

    def close(self) -> None:
        if self._ctx:
            self._lib.nya_compute_free(self._ctx)
            self._ctx = None
            self._borrowed.clear()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def name(self) -> str:
        return self._lib.nya_compute_name(self._ctx).decode()

    @property
    def capabilities(self) -> int:
        return self._lib.nya_compute_capabilities(self._ctx)

    def stats(self) -> dict:
        s = ComputeStats()
        self._lib.nya_compute_context_stats(self._ctx, ctypes.byref(s))
        return s.as_dict()

    def matmul_typed(self, weights: np.ndarray, rows: int, cols: int, type_id: int, x: np.ndarray,
                     batch: int, out: np.ndarray | None = None) -> np.ndarray:
        """Y[batch][rows] = X[batch][cols] . W^T through nya_compute_matmul_typed."""
        w = np.ascontiguousarray(weights)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        if x.size != batch * cols:
            raise ValueError("x must hold batch*cols floats")
        if out is None:
            out = np.empty(batch * rows, dtype=np.float32)
        self._borrowed.append(w)
        status = self._lib.nya_compute_matmul_typed(self._ctx, w.ctypes.data, rows, cols, type_id,
                                                    _float_ptr(x), _float_ptr(out), batch)
        if status != 0:
            raise ComputeDeclined(f"matmul declined (type {type_id}, {rows}x{cols}, batch {batch}); "
                                  f"provider now reports {self.name!r}")
        return out.reshape(batch, rows)

    def matvec_typed(self, weights: np.ndarray, rows: int, cols: int, type_id: int, x: np.ndarray) -> np.ndarray:
        w = np.ascontiguousarray(weights)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        out = np.empty(rows, dtype=np.float32)
        self._borrowed.append(w)
        status = self._lib.nya_compute_matvec_typed(self._ctx, w.ctypes.data, rows, cols, type_id,
                                                    _float_ptr(x), _float_ptr(out))
        if status != 0:
            raise ComputeDeclined(f"matvec declined (type {type_id}, {rows}x{cols}); provider now reports {self.name!r}")
        return out

"""ctypes access to the HIP runtime and to libfyodor_hip.so's C ABI.

Used by the benchmark to hold weights resident in HBM and to time kernels
with HIP events recorded on the stream the kernels are launched on.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from . import KERNEL_LIBRARY

_vp, _sz, _u = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint
_up = ctypes.c_size_t  # uintptr_t


class HipError(RuntimeError):
    pass


class Runtime:
    H2D, D2H, D2D = 1, 2, 3

    def __init__(self, library: str = "libamdhip64.so"):
        self.lib = ctypes.CDLL(library)
        L = self.lib
        L.hipMalloc.argtypes = [ctypes.POINTER(_vp), _sz]
        L.hipFree.argtypes = [_vp]
        L.hipMemcpy.argtypes = [_vp, _vp, _sz, ctypes.c_int]
        L.hipMemcpyAsync.argtypes = [_vp, _vp, _sz, ctypes.c_int, _vp]
        L.hipMemsetAsync.argtypes = [_vp, ctypes.c_int, _sz, _vp]
        L.hipStreamCreateWithFlags.argtypes = [ctypes.POINTER(_vp), _u]
        L.hipStreamDestroy.argtypes = [_vp]
        L.hipStreamSynchronize.argtypes = [_vp]
        L.hipEventCreate.argtypes = [ctypes.POINTER(_vp)]
        L.hipEventDestroy.argtypes = [_vp]
        L.hipEventRecord.argtypes = [_vp, _vp]
        L.hipEventSynchronize.argtypes = [_vp]
        L.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), _vp, _vp]
        L.hipGetErrorString.restype = ctypes.c_char_p
        L.hipGetErrorString.argtypes = [ctypes.c_int]
        L.hipMemGetInfo.argtypes = [ctypes.POINTER(_sz), ctypes.POINTER(_sz)]
        L.hipDeviceGetName.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int]
        L.hipDeviceGetAttribute.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int]
        self.check(L.hipSetDevice(0), "hipSetDevice")

    def check(self, status: int, what: str) -> None:
        if status != 0:
            raise HipError(f"{what} failed: {status} {self.lib.hipGetErrorString(status).decode()}")

    def malloc(self, nbytes: int) -> int:
        p = _vp()
        self.check(self.lib.hipMalloc(ctypes.byref(p), max(nbytes, 1)), "hipMalloc")
        return p.value

    def free(self, p: int) -> None:
        self.check(self.lib.hipFree(p), "hipFree")

    def upload(self, dst: int, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        self.check(self.lib.hipMemcpy(dst, a.ctypes.data, a.nbytes, self.H2D), "hipMemcpy H2D")

    def download(self, src: int, out: np.ndarray) -> np.ndarray:
        self.check(self.lib.hipMemcpy(out.ctypes.data, src, out.nbytes, self.D2H), "hipMemcpy D2H")
        return out

    def stream(self) -> int:
        s = _vp()
        self.check(self.lib.hipStreamCreateWithFlags(ctypes.byref(s), 1), "hipStreamCreateWithFlags")
        return s.value

    def sync(self, stream: int) -> None:
        self.check(self.lib.hipStreamSynchronize(stream), "hipStreamSynchronize")

    def event(self) -> int:
        e = _vp()
        self.check(self.lib.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        return e.value

    def record(self, event: int, stream: int) -> None:
        self.check(self.lib.hipEventRecord(event, stream), "hipEventRecord")

    def elapsed_ms(self, start: int, end: int) -> float:
        self.check(self.lib.hipEventSynchronize(end), "hipEventSynchronize")
        ms = ctypes.c_float()
        self.check(self.lib.hipEventElapsedTime(ctypes.byref(ms), start, end), "hipEventElapsedTime")
        return ms.value

    def device_name(self) -> str:
        buf = ctypes.create_string_buffer(256)
        self.check(self.lib.hipDeviceGetName(buf, 256, 0), "hipDeviceGetName")
        return buf.value.decode()

    def attribute(self, attr: int) -> int:
        v = ctypes.c_int()
        self.check(self.lib.hipDeviceGetAttribute(ctypes.byref(v), attr, 0), "hipDeviceGetAttribute")
        return v.value


class Kernels:
    """libfyodor_hip.so (include/fyodor_hip.h)."""

    def __init__(self, path: Path = KERNEL_LIBRARY):
        if not Path(path).exists():
            raise FileNotFoundError(f"{path} is missing: run `python -m fyodor_amd.build`")
        self.lib = ctypes.CDLL(str(path))
        L = self.lib
        L.nya_hip_abi_version.restype = _u
        L.nya_hip_weight_bytes.argtypes = [_u, _sz, _sz, ctypes.POINTER(_sz)]
        L.nya_hip_weight_layout.argtypes = [_u]
        L.nya_hip_weight_pack.argtypes = [_vp, _vp, _u, _sz, _sz]
        L.nya_hip_workspace_bytes.argtypes = [_u, _sz, _sz, _sz, ctypes.POINTER(_sz)]
        L.nya_hip_matmul.argtypes = [_up, _u, _sz, _sz, _up, _up, _sz, _up, _sz, _up]
        L.nya_hip_matmul_static.argtypes = [_up, _u, _sz, _sz, _up, _up, _sz, _up]
        L.nya_hip_copy.argtypes = [_up, _up, _sz, _up]
        L.nya_hip_read.argtypes = [_up, _sz, _up, _up]
        L.nya_hip_read_shaped.argtypes = [_up, _sz, _up, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _up]
        L.nya_hip_kernel_name.restype = ctypes.c_char_p
        L.nya_hip_kernel_name.argtypes = [_u, _sz, _sz, _sz]

    def device_weights(self, w: np.ndarray, type_id: int, rows: int, cols: int) -> np.ndarray:
        """GGUF bytes -> the device layout (host side)."""
        layout = self.lib.nya_hip_weight_layout(type_id)
        if layout < 0:
            raise ValueError(f"type {type_id} unsupported")
        if layout == 0:
            return w
        out = np.empty_like(w)
        if self.lib.nya_hip_weight_pack(out.ctypes.data, w.ctypes.data, type_id, rows, cols):
            raise ValueError("nya_hip_weight_pack declined")
        return out

    def workspace_bytes(self, type_id: int, rows: int, cols: int, batch: int) -> int:
        b = _sz()
        if self.lib.nya_hip_workspace_bytes(type_id, rows, cols, batch, ctypes.byref(b)):
            raise ValueError("request unsupported")
        return b.value

    def matmul(self, w: int, type_id: int, rows: int, cols: int, x: int, y: int, batch: int,
               workspace: int, workspace_bytes: int, stream: int) -> None:
        status = self.lib.nya_hip_matmul(w, type_id, rows, cols, x, y, batch, workspace, workspace_bytes, stream)
        if status != 0:
            raise HipError(f"nya_hip_matmul returned {status}")

    def matmul_static(self, w: int, type_id: int, rows: int, cols: int, x: int, y: int, batch: int,
                      stream: int) -> None:
        """The allocation-free entry point (scratch in the library's static
        device array)."""
        status = self.lib.nya_hip_matmul_static(w, type_id, rows, cols, x, y, batch, stream)
        if status != 0:
            raise HipError(f"nya_hip_matmul_static returned {status}")

    def copy(self, dst: int, src: int, nbytes: int, stream: int) -> None:
        status = self.lib.nya_hip_copy(dst, src, nbytes, stream)
        if status != 0:
            raise HipError(f"nya_hip_copy returned {status}")

    def read(self, src: int, nbytes: int, sink: int, stream: int) -> None:
        """Plain streaming read of nbytes (diagnostic HBM read ceiling)."""
        status = self.lib.nya_hip_read(src, nbytes, sink, stream)
        if status != 0:
            raise HipError(f"nya_hip_read returned {status}")

    def read_shaped(self, src: int, nbytes: int, sink: int, waves: int, depth: int, per_cu: int, mode: int,
                    stream: int) -> None:
        """The plain read in another shape (waves x depth, workgroups per CU,
        0 non-temporal / 1 default policy / 2 into LDS)."""
        status = self.lib.nya_hip_read_shaped(src, nbytes, sink, waves, depth, per_cu, mode, stream)
        if status != 0:
            raise HipError(f"nya_hip_read_shaped returned {status}")

    def kernel_name(self, type_id: int, rows: int, cols: int, batch: int) -> str:
        name = self.lib.nya_hip_kernel_name(type_id, rows, cols, batch)
        return name.decode() if name else ""


class Graph:
    """A captured sequence of launches on one stream (hipGraph)."""

    def __init__(self, rt: Runtime, stream: int, launches):
        L = rt.lib
        vp = ctypes.c_void_p
        L.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
        L.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
        L.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, vp, ctypes.c_size_t]
        L.hipGraphLaunch.argtypes = [vp, vp]
        L.hipGraphExecDestroy.argtypes = [vp]
        L.hipGraphDestroy.argtypes = [vp]
        self.rt, self.stream = rt, stream
        rt.check(L.hipStreamBeginCapture(stream, 0), "hipStreamBeginCapture")
        try:
            for launch in launches:
                launch()
        finally:
            graph = vp()
            rt.check(L.hipStreamEndCapture(stream, ctypes.byref(graph)), "hipStreamEndCapture")
        self.graph = graph
        self.exec = vp()
        rt.check(L.hipGraphInstantiate(ctypes.byref(self.exec), graph, None, None, 0), "hipGraphInstantiate")

    def launch(self):
        self.rt.check(self.rt.lib.hipGraphLaunch(self.exec, self.stream), "hipGraphLaunch")

    def close(self):
        self.rt.lib.hipGraphExecDestroy(self.exec)
        self.rt.lib.hipGraphDestroy(self.graph)

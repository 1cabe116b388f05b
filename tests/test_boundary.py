"""The C-ABI boundary on the CPU: both native libraries load and export every
function their public headers declare, the host-side queries answer as
documented, and the weight packer is the byte permutation the device layout
specifies (fyodor_amd/csrc/formats.h). Nothing here launches GPU work."""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from fyodor_amd import BF16, F16, F32, KERNEL_LIBRARY, PROVIDER_LIBRARY, Q4_0, Q4_K, Q6_K, Q8_0, storage_bytes, synth
from fyodor_amd.hip import Kernels

INCLUDE = Path(__file__).resolve().parent.parent / "include"


def declared(header: str) -> set:
    text = (INCLUDE / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(nya_[a-z0-9_]+)\s*\(", text))


def exported(lib: Path) -> set:
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_kernel_library_exports_its_header():
    want = declared("fyodor_hip.h")
    assert want == {"nya_hip_abi_version", "nya_hip_weight_bytes", "nya_hip_weight_layout", "nya_hip_weight_pack",
                    "nya_hip_workspace_bytes", "nya_hip_matmul", "nya_hip_kernel_name", "nya_hip_copy"}
    assert want <= exported(KERNEL_LIBRARY)


def test_provider_library_exports_compute_api():
    want = declared("compute.h") | declared("compute_backend.h")
    assert "nya_rocm_backend" in want and "nya_compute_matmul_typed" in want
    missing = want - exported(PROVIDER_LIBRARY)
    assert not missing, missing


def test_provider_needs_no_rocm_link():
    """The C provider resolves HIP at run time (rocm/rocm.c:155-166)."""
    out = subprocess.run(["ldd", str(PROVIDER_LIBRARY)], capture_output=True, text=True).stdout
    assert "amdhip64" not in out and "fyodor_hip" not in out


@pytest.fixture(scope="module")
def kernels():
    return Kernels()


def test_queries(kernels):
    L = kernels.lib
    assert L.nya_hip_abi_version() == 1
    b = ctypes.c_size_t()
    for t, block, size in [(F32, 1, 4), (F16, 1, 2), (BF16, 1, 2), (Q4_0, 32, 18), (Q8_0, 32, 34),
                           (Q4_K, 256, 144), (Q6_K, 256, 210)]:
        assert L.nya_hip_weight_bytes(t, 3, 4 * block, ctypes.byref(b)) == 0 and b.value == 3 * 4 * size
        assert L.nya_hip_weight_bytes(t, 3, 4 * block + (block > 1), ctypes.byref(b)) == (1 if block > 1 else 0)
        assert L.nya_hip_weight_layout(t) == (0 if block == 1 else 1)
        assert L.nya_hip_workspace_bytes(t, 3, 4 * block, 2, ctypes.byref(b)) == 0
    assert L.nya_hip_weight_bytes(99, 3, 32, ctypes.byref(b)) == 1 and L.nya_hip_weight_layout(99) == -1
    assert L.nya_hip_weight_bytes(Q8_0, 0, 32, ctypes.byref(b)) == 1
    assert L.nya_hip_weight_bytes(Q8_0, 1 << 31, 32, ctypes.byref(b)) == 1
    assert L.nya_hip_matmul(0, Q8_0, 3, 32, 16, 16, 1, 0, 0, 0) == 1          # declined, nothing enqueued
    assert kernels.kernel_name(Q4_K, 14336, 4096, 1) == "quant_rows"


def unpack_reference(dev: np.ndarray, t: int, rows: int, cols: int) -> np.ndarray:
    """Inverse of the device layout, written from its specification."""
    out = np.empty(storage_bytes(t, rows, cols), dtype=np.uint8)
    if t in (Q8_0, Q4_0):
        n = rows * cols // 32
        q = 32 if t == Q8_0 else 16
        blk = out.reshape(n, q + 2)
        blk[:, 0:2] = dev[q * n:].reshape(n, 2)
        blk[:, 2:18] = dev[:16 * n].reshape(n, 16)
        if t == Q8_0:
            blk[:, 18:34] = dev[16 * n:32 * n].reshape(n, 16)
    elif t == Q4_K:
        U, ns = cols // 64, cols // 256
        n = rows * U
        qa, qb = dev[:16 * n].reshape(rows, ns, 4, 16), dev[16 * n:32 * n].reshape(rows, ns, 4, 16)
        sl = dev[32 * n:].view(np.uint32).reshape(rows, ns, 4)
        blk = out.reshape(rows, ns, 144)
        for p in range(4):
            blk[:, :, 16 + 32 * p:32 + 32 * p] = qa[:, :, p]
            blk[:, :, 32 + 32 * p:48 + 32 * p] = qb[:, :, p]
            blk[:, :, p] = (sl[:, :, p] >> 24).astype(np.uint8)
        sc = [(sl[:, :, g // 2] >> (12 * (g % 2))) & 63 for g in range(8)]
        mn = [(sl[:, :, g // 2] >> (12 * (g % 2) + 6)) & 63 for g in range(8)]
        for g in range(4):
            blk[:, :, 4 + g] = sc[g] | ((sc[g + 4] >> 4) << 6)
            blk[:, :, 8 + g] = mn[g] | ((mn[g + 4] >> 4) << 6)
            blk[:, :, 12 + g] = (sc[g + 4] & 15) | ((mn[g + 4] & 15) << 4)
    else:
        ns = cols // 256
        U, n = 4 * ns, rows * cols // 64
        a, b, c = (dev[i * 16 * n:(i + 1) * 16 * n].reshape(rows, ns, 2, 2, 16) for i in range(3))
        sc = dev[48 * n:52 * n].reshape(rows, ns, 2, 2, 4)
        d = dev[52 * n:].reshape(rows, ns, 2)
        blk = out.reshape(rows, ns, 210)
        for h in range(2):
            for l16 in range(2):
                blk[:, :, 64 * h + 16 * l16:64 * h + 16 * l16 + 16] = a[:, :, h, l16]
                blk[:, :, 64 * h + 32 + 16 * l16:64 * h + 48 + 16 * l16] = b[:, :, h, l16]
                blk[:, :, 128 + 32 * h + 16 * l16:128 + 32 * h + 16 * l16 + 16] = c[:, :, h, l16]
                for q in range(4):
                    blk[:, :, 192 + 8 * h + 2 * q + l16] = sc[:, :, h, l16, q]
        blk[:, :, 208:210] = d
    return out


@pytest.mark.parametrize("t", [Q4_0, Q8_0, Q4_K, Q6_K])
def test_pack_is_the_specified_permutation(kernels, t):
    rows, cols = 5, 1024
    w = synth.weights(t, rows, cols, 21)   # random scale bytes: every 12-byte pattern
    dev = kernels.device_weights(w, t, rows, cols)
    assert dev.nbytes == w.nbytes and not np.shares_memory(dev, w)
    assert np.array_equal(unpack_reference(dev, t, rows, cols), w)


def test_gemm_dispatch_and_workspace():
    """Batches above 8 of the quantized types ask for the activation pieces'
    workspace and name the MFMA GEMM; dense types and small batches need
    none (nothing is launched)."""
    kern = Kernels()
    for t in (Q4_0, Q8_0, Q4_K, Q6_K):
        assert kern.workspace_bytes(t, 4096, 4096, 8) == 0
        assert kern.workspace_bytes(t, 4096, 4096, 9) == 6 * 4096 * 9
        assert kern.workspace_bytes(t, 4096, 4096, 512) == 6 * 4096 * 512
        assert kern.kernel_name(t, 4096, 4096, 512) == "gemm_tile"
        assert kern.kernel_name(t, 4096, 4096, 8) != "gemm_tile"
    for t in (F32, BF16):
        assert kern.workspace_bytes(t, 4096, 4096, 512) == 0
        assert kern.kernel_name(t, 4096, 4096, 512) == "skinny_dense"

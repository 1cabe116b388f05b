"""Builds the in-tree native libraries.

- ``fyodor_amd/lib/libfyodor_hip.so``: gfx950 kernels + their C ABI (hipcc).
- ``fyodor_amd/lib/libfyodor_rocm.so``: the C provider (rocm.c) with the
  compute dispatch and vendor glue it links against (gcc, no ROCm headers).

Run ``python -m fyodor_amd.build``. Every call recompiles.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent
REPO = ROOT.parent
LIB = ROOT / "lib"
CSRC = ROOT / "csrc"
HIP_SOURCES = ["abi.hip", "dense.hip", "smalln.hip", "matvec.hip", "prefill.hip", "prefill_f16.hip", "resident.hip",
               "pack.cpp"]
C_SOURCES = ["core/compute.c", "core/vendor.c", "rocm/rocm.c"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
    # Packed FP32 arithmetic is kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# Per-source additions. The int8 block-dot kernels read every MFMA result at
# once in VALU code: results in VGPRs (not AGPRs) save a copy per register.
EXTRA_FLAGS = {f: ["-mllvm", "-amdgpu-mfma-vgpr-form"] for f in ("smalln.hip", "matvec.hip", "prefill.hip", "prefill_f16.hip")}
C_FLAGS = [
    "-std=c17", "-O2", "-fPIC", "-Wall", "-Wextra", "-Wpedantic", "-Wshadow",
    "-D_POSIX_C_SOURCE=200809L",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    noise = [l for l in proc.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip()]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the gfx950 kernel library cannot be built")
    return path


def build_kernels() -> Path:
    LIB.mkdir(exist_ok=True)
    obj_dir = LIB / "obj"
    obj_dir.mkdir(exist_ok=True)
    sources = [CSRC / s for s in HIP_SOURCES if (CSRC / s).exists()]
    objects = [obj_dir / (s.stem + ".o") for s in sources]
    cc = hipcc()
    inc = [f"-I{REPO / 'include'}", f"-I{CSRC}"]

    def compile_one(pair):
        src, obj = pair
        lang = ["-x", "hip"] if src.suffix == ".hip" else []
        _run([cc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), *inc, *lang, "-c", str(src), "-o", str(obj)])

    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        list(pool.map(compile_one, zip(sources, objects)))
    out = LIB / "libfyodor_hip.so"
    tmp = LIB / "libfyodor_hip.so.tmp"
    _run([cc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)])
    os.replace(tmp, out)
    return out


def build_provider() -> Path:
    LIB.mkdir(exist_ok=True)
    out = LIB / "libfyodor_rocm.so"
    tmp = LIB / "libfyodor_rocm.so.tmp"
    _run(["gcc", *C_FLAGS, f"-I{REPO / 'include'}", f"-I{ROOT / 'core'}", f"-I{ROOT / 'rocm'}",
          *[str(ROOT / s) for s in C_SOURCES], "-shared", "-ldl", "-lm", "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_all() -> None:
    build_provider()
    build_kernels()


if __name__ == "__main__":
    build_all()
    print("built", LIB / "libfyodor_hip.so", "and", LIB / "libfyodor_rocm.so")

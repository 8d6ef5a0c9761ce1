"""Build of the native library ``aklr_amd/libaklr_amd.so`` from ``aklr_amd/csrc/*.hip`` with hipcc.

In-tree build for gfx950 only: every ``.hip`` file compiles to an object in ``aklr_amd/_build/`` (in
parallel), then hipcc links them into one shared library exporting the C ABI of
``include/aklr_amd.h``. Mirrors the role of aklr/core/jit/hip_extension.py (hipcc, ``-O3``, one arch),
without torch in the loop: the library has no torch types in its interface.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD_DIR = PKG / "_build"
LIB_PATH = PKG / "libaklr_amd.so"
ARCH = "gfx950"

# Packed-fp32 VALU ops are switched off: the kernels' fp32 arithmetic stays scalar per lane. The sources
# also switch them off themselves (AKLR_SCALAR_FP32_BEGIN/END), for builds that pass no such flag.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the aklr_amd native library needs ROCm's hipcc to build")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every kernel source and link ``libaklr_amd.so``; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(srcs), max(1, (os.cpu_count() or 4) // 2), 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)

"""ctypes binding of the native library (the C ABI declared in include/aklr_amd.h).

The library is loaded once per process, on first use. A missing library is an error, never a
silent fallback: every op raises ``NativeLibraryError`` when asked to run without it.
"""
from __future__ import annotations

import ctypes
import hashlib
import threading
from pathlib import Path

from ._build import LIB_PATH

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_size = ctypes.c_size_t
_vp = ctypes.c_void_p

# name -> (restype, argtypes); keep in the order of include/aklr_amd.h
SIGNATURES: dict[str, tuple] = {
    "aklr_abi_version": (_c_int, []),
    "aklr_status_string": (ctypes.c_char_p, [_c_int]),
    "aklr_per_group_quant_fp8": (_c_int, [_vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _vp]),
    "aklr_per_group_quant_mxfp8": (_c_int, [_vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _vp]),
    "aklr_dynamic_mxfp4_quant": (_c_int, [_vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _c_int, _vp]),
    "aklr_gemm_a8w8_blockscale_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64]),
    "aklr_gemm_a8w8_blockscale_kernel": (_c_int, [_c_i64, _c_i64, _c_i64, _c_int]),
    "aklr_gemm_a8w8_blockscale": (
        _c_int,
        [_vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_int, _c_int, _c_int, _vp, _c_size, _vp],
    ),
    "aklr_gemm_a8w8_blockscale_noalloc": (
        _c_int,
        [_vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_int, _c_int, _c_int, _vp],
    ),
    "aklr_noalloc_scratch": (_c_int, [ctypes.POINTER(_vp), ctypes.POINTER(_c_size)]),
    "aklr_transpose_b8": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _vp]),
    "aklr_quant_gemm_a8w8_blockscale_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64]),
    "aklr_quant_gemm_a8w8_blockscale_fused": (_c_int, [_c_i64, _c_i64, _c_i64]),
    "aklr_quant_gemm_a8w8_blockscale": (
        _c_int,
        [_vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _vp,
         _c_size, _vp],
    ),
    "aklr_gemm_a4w4_mxfp4_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64]),
    "aklr_gemm_a4w4_mxfp4": (
        _c_int,
        [_vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_int,
         _c_int, _c_int, _vp, _c_size, _vp],
    ),
    "aklr_moe_fp8_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "aklr_deepseek_v2_fp8_moe": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int,
         ctypes.c_float, _c_int, _vp, _vp, _c_size, _vp],
    ),
    "aklr_moe_fp8_route": (
        _c_int,
        [_vp, _vp, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, ctypes.c_float, _c_int, _vp, _vp, _vp],
    ),
    "aklr_moe_fp8_experts": (
        _c_int,
        [_vp, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _vp, _c_i64, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _c_size, _vp],
    ),
    "aklr_probe_hbm_read": (_c_int, [_vp, _c_i64, _vp, _c_int, _c_int, _vp]),
}

# enums of include/aklr_amd.h
AKLR_OK = 0
AKLR_ERR_INVALID_ARGUMENT, AKLR_ERR_UNSUPPORTED, AKLR_ERR_WORKSPACE, AKLR_ERR_LAUNCH = 1, 2, 3, 4
AKLR_ERR_SCRATCH_LIMIT = 5
NOALLOC_SCRATCH_BYTES = 48 << 20  # AKLR_NOALLOC_SCRATCH_BYTES
FP8_E4M3FN, FP8_E5M2 = 0, 1
OUT_BF16, OUT_F16 = 0, 1
B_ROW_MAJOR, B_PRESHUFFLE_16x16 = 0, 1
SCALES_ROW_MAJOR, SCALES_SHUFFLED = 0, 1
ABI_VERSION = 1


class NativeLibraryError(RuntimeError):
    """The HIP library is missing, stale, or a call into it failed."""


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_digest: str | None = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises NativeLibraryError when it is not built."""
    global _lib, _digest
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = Path(LIB_PATH)
            if not path.exists():
                raise NativeLibraryError(
                    f"{path} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
                    "(or `python -m aklr_amd._build`); the GPU path has no fallback"
                )
            handle = ctypes.CDLL(str(path))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            if handle.aklr_abi_version() != ABI_VERSION:
                raise NativeLibraryError("libaklr_amd.so ABI version does not match the Python binding")
            _digest = hashlib.sha256(path.read_bytes()).hexdigest()[:16]
            _lib = handle
    return _lib


def digest() -> str:
    lib()
    assert _digest is not None
    return _digest


def check(status: int, what: str) -> None:
    if status != AKLR_OK:
        msg = lib().aklr_status_string(status).decode()
        raise NativeLibraryError(f"{what}: {msg} (status {status})")

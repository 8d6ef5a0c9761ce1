"""The C-ABI library without a GPU: it loads, exports every entry point include/aklr_amd.h declares
(unmangled), matches the Python binding's table, and rejects invalid arguments before any launch."""
from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

from aklr_amd import _build, _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "aklr_amd.h"


def declared() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(aklr_\w+)\s*\(", text))


def test_header_declares_the_binding_table():
    assert declared() == set(_lib.SIGNATURES)


def test_every_declared_symbol_is_exported(native_lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(_build.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = declared() - exported
    assert not missing, f"not exported (or C++-mangled): {sorted(missing)}"
    for name in declared():
        assert hasattr(native_lib, name)


def test_version_and_status_strings(native_lib):
    assert native_lib.aklr_abi_version() == _lib.ABI_VERSION
    assert native_lib.aklr_status_string(0) == b"ok"
    assert native_lib.aklr_status_string(1) == b"invalid argument"
    assert native_lib.aklr_status_string(3) == b"workspace too small"
    assert native_lib.aklr_status_string(99) == b"unknown status"


def test_invalid_arguments_rejected_before_launch(native_lib):
    L = native_lib
    buf = ctypes.create_string_buffer(1 << 16)
    p = ctypes.addressof(buf)
    p16 = (p + 15) & ~15
    # null pointers
    assert L.aklr_per_group_quant_fp8(None, 128, p16, p16, 1, 128, None) == 1
    # hidden size not a multiple of 128 / 32
    assert L.aklr_per_group_quant_fp8(p16, 100, p16, p16, 1, 100, None) == 1
    assert L.aklr_per_group_quant_mxfp8(p16, 48, p16, p16, 1, 48, None) == 1
    assert L.aklr_dynamic_mxfp4_quant(p16, 64, p16, p16, 1, 64, 7, None) == 2  # unknown scale layout
    # misaligned x
    assert L.aklr_per_group_quant_fp8(p16 + 2, 128, p16, p16, 1, 128, None) == 1
    # zero tokens: nothing to launch
    assert L.aklr_per_group_quant_fp8(p16, 128, p16, p16, 0, 128, None) == 0
    # GEMM: k % 128, n % 16, dtype and layout enums
    args = lambda m, n, k, dt=0, lay=0: (p16, k, p16, k, p16, k // 128 or 1, 1, p16, max(k // 128, 1), None, p16, n,
                                         m, n, k, dt, lay, 0, None, 0, None)
    assert L.aklr_gemm_a8w8_blockscale(*args(4, 16, 100)) == 1
    assert L.aklr_gemm_a8w8_blockscale(*args(4, 20, 128)) == 1
    assert L.aklr_gemm_a8w8_blockscale(*args(4, 16, 128, dt=5)) == 2
    assert L.aklr_gemm_a8w8_blockscale(*args(4, 16, 128, lay=9)) == 2
    assert L.aklr_gemm_a8w8_blockscale(*args(0, 16, 128)) == 0
    a4 = lambda m, n, k: (p16, k // 2, p16, k // 2, p16, k // 32, p16, k // 32, None, p16, n, m, n, k, 0, 0, 0, None,
                          0, None)
    assert L.aklr_gemm_a4w4_mxfp4(*a4(4, 16, 96)) == 1
    assert L.aklr_gemm_a4w4_mxfp4(*a4(0, 16, 64)) == 0


def test_workspace_sizes_are_host_computable(native_lib):
    L = native_lib
    assert L.aklr_gemm_a8w8_blockscale_workspace_bytes(0, 16, 128) == 0
    up = lambda x, q: -(-x // q) * q
    for m, n, k in ((1, 2112, 7168), (16, 7168, 16384), (4096, 7168, 16384), (128, 24576, 1536), (256, 2112, 7168)):
        ws = L.aklr_gemm_a8w8_blockscale_workspace_bytes(m, n, k)
        # 128 KiB of split-K arrival words plus at most 8 splits of fp32 partials over whole 16x16 tiles
        # of workgroups at most 256 x 256
        assert ws % 1024 == 0 and ws <= 131072 + 8 * up(m, 256) * up(n, 256) * 4
    assert L.aklr_gemm_a4w4_mxfp4_workspace_bytes(1, 10240, 8192) % 4 == 0


def test_gemm8_kernel_query(native_lib):
    # 0: the stream kernel, 1: the LDS kernel, as aklr_gemm_a8w8_blockscale plans (m, n, k) for a layout
    q, row, pre = native_lib.aklr_gemm_a8w8_blockscale_kernel, _lib.B_ROW_MAJOR, _lib.B_PRESHUFFLE_16x16
    assert q(1, 2112, 7168, row) == 0 and q(128, 24576, 1536, pre) == 0 and q(300, 1024, 2048, row) == 1
    # row blocks (preshuffled): m = 65..128 on K <= 64 blocks, m = 129..256 on K <= 16, m = 257..1024 on
    # 16..32 K blocks while they make <= 256 workgroups; row-major weights at m = 65..128 on K <= 16 blocks:
    # 64x64 LDS tiles
    assert q(300, 1024, 2048, pre) == 0 and q(1024, 1536, 4096, pre) == 0 and q(1024, 1536, 4096, row) == 1
    assert q(1024, 2112, 4096, pre) == 1 and q(1024, 1536, 8192, pre) == 1 and q(1025, 512, 4096, pre) == 1
    assert q(1024, 1536, 1024, pre) == 1
    assert q(128, 4096, 8192, pre) == 0 and q(128, 4096, 8192, row) == 0
    assert q(128, 7168, 2048, pre) == 0 and q(128, 7168, 2048, row) == 1 and q(64, 7168, 2048, row) == 0
    assert q(256, 7168, 2048, pre) == 0 and q(256, 7168, 2048, row) == 1 and q(256, 2112, 7168, pre) == 1
    assert q(257, 7168, 2048, pre) == 1 and q(256, 24576, 1536, pre) == 1
    assert q(0, 16, 128, row) == -1 and q(4, 16, 100, row) == -1 and q(4, 16, 128, 7) == -1


def test_quant_gemm_path_and_workspace_are_host_computable(native_lib):
    L = native_lib
    fused = L.aklr_quant_gemm_a8w8_blockscale_fused
    # one launch at one row tile on the decode shapes of up to 56 K blocks; two kernels past 16 rows, on a
    # wave-split-K plan (4096 x 8192), on the long-K plan (7168 x 16384, whose GEMM walks K in its own
    # order) and for empty sizes
    assert fused(16, 2112, 7168) == 1 and fused(1, 2112, 7168) == 1 and fused(4, 24576, 1536) == 1
    assert fused(16, 4096, 16384) == 1
    assert fused(17, 7168, 16384) == 0 and fused(300, 1024, 2048) == 0
    assert fused(1, 4096, 8192) == 0 and fused(1, 7168, 16384) == 0 and fused(16, 7168, 16384) == 0
    assert fused(0, 7168, 16384) == 0 and fused(1, 7168, 64) == 0
    # the two-kernel path stages the codes and scales past the 128 KiB arrival-word region
    m, n, k = 20, 2112, 128
    assert L.aklr_quant_gemm_a8w8_blockscale_workspace_bytes(m, n, k) >= 131072 + m * k + (k // 128) * m * 4


def test_every_plan_fits_the_noalloc_scratch(native_lib):
    # aklr_gemm_a8w8_blockscale_noalloc serves a plan only when its workspace fits the library's scratch
    # array; the planner splits K only while the workgroups stay about one round (<= 256), which bounds
    # every plan's scratch below the array: a sweep over m, n, k finds none larger
    L = native_lib
    worst = 0
    for m in (1, 4, 16, 17, 32, 64, 100, 128, 129, 200, 256, 300, 512, 1024, 2048, 4096, 8192, 2**20):
        for n in (16, 48, 144, 1024, 1920, 2112, 4096, 7168, 24576, 65536, 262144):
            for k in (128, 512, 2048, 7168, 16384, 65536):
                worst = max(worst, L.aklr_gemm_a8w8_blockscale_workspace_bytes(m, n, k))
    assert 0 < worst <= _lib.NOALLOC_SCRATCH_BYTES

"""GPU parity of the 128x128-block-scaled FP8 GEMM and the MXFP4 GEMM against the CPU oracle.

Tolerance (written here, as the north star states it): |out - y| <= 1e-2 * rms(y) + 1e-2 * |y| per
element, y the oracle's fp32 result (dequantize to fp32, then matmul); the contract's own
ToleranceBound (atol 1e-2, rtol 1e-2 + bf16 unit roundoff) is checked too for FP8.
Full outputs are compared up to decode sizes; prefill sizes compare a seeded sample of rows x columns
(the oracle computes exactly those) plus size-independent properties (determinism, linearity in the
scales). test_gpu_full_outputs.py compares every output at prefill sizes, against a float32
restatement on the GPU that is itself pinned to the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import aklr_amd
from aklr_amd import layouts, workloads
from oracle import gemm as ogemm
from oracle import quant as oquant
from tests.helpers import bf16_bits, f32, say, u8

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _fp8_inputs(m, n, k, seed=0, dtype=torch.float8_e4m3fn):
    x = workloads.activations(m, k, seed=seed, device=DEV)
    if k <= 21504:
        q, s = aklr_amd.per_group_quant_fp8(x)
    else:  # past per_group_quant_fp8's hidden-size contract: codes and scales from the oracle
        q_np, s_np = oquant.per_group_quant_fp8(bf16_bits(x))
        q = torch.from_numpy(q_np).view(torch.float8_e4m3fn).to(DEV)
        s = torch.from_numpy(s_np).to(DEV)
    b, bs = workloads.blockwise_fp8_weight(n, k, seed=seed + 1, device=DEV)
    if dtype == torch.float8_e5m2:
        q = q.float().to(torch.float8_e5m2)
        b = b.float().to(torch.float8_e5m2)
    return q, s, b, bs


def _sample(m, n, rows, cols, seed=0):
    rng = np.random.default_rng(seed)
    r = np.arange(m) if m <= rows else np.sort(rng.choice(m, rows, replace=False))
    c = np.arange(n) if n <= cols else np.sort(rng.choice(n, cols, replace=False))
    return r, c


def _check(out, ref, what, contract=True, out_dtype="bfloat16"):
    got = f32(out) if isinstance(out, torch.Tensor) else out
    err, rms = ogemm.rms_normalized_error(got, ref)
    assert ogemm.within_north_star(got, ref), f"{what}: max|err|/rms {err:.3e} outside tolerance"
    if contract:
        assert ogemm.within_contract_tolerance(got, ref, out_dtype), f"{what}: contract ToleranceBound exceeded"


def _fmt(dtype):
    return "e5m2" if dtype == torch.float8_e5m2 else "e4m3fn"


def _run_and_check(m, n, k, *, variant="row_major", mode="K", bias=False, out_dtype=None, seed=0,
                   dtype=torch.float8_e4m3fn, rows=64, cols=512):
    say(f"gemm_a8w8 m={m} n={n} k={k} variant={variant} mode={mode} bias={bias} out={out_dtype} {_fmt(dtype)}")
    q, s, b, bs = _fp8_inputs(m, n, k, seed, dtype)
    bias_t = (torch.randn(n, device=DEV, generator=workloads.generator(seed + 7, DEV)) if bias else None)
    kwargs = {}
    if variant == "row_major":
        a_scale = s.t().contiguous() if mode == "K" else s
        bb = b
    else:
        bb = layouts.shuffle_weight(b)
        kwargs["operand_format"] = "none:preshuffled"
        if variant == "b_shuffled":
            a_scale = s.view(m, k // 128)  # the group-major bytes, read column-major
        else:
            a_scale = s.t().contiguous()
            a_scale.is_row_major = True
    out = aklr_amd.gemm_a8w8_blockwise_scaled(q, bb, a_scale, bs, scale_major_mode=mode, bias=bias_t,
                                              out_dtype=out_dtype, **kwargs)
    assert isinstance(out, torch.Tensor), f"not served: {out}"
    torch.cuda.synchronize()
    r, c = _sample(m, n, rows, cols, seed)
    s_np = s.cpu().numpy()  # (kb, m)
    ref = ogemm.gemm_a8w8_blockwise_scaled(u8(q), u8(b), s_np, bs.cpu().numpy(), fmt=_fmt(dtype),
                                           scale_major_mode="MN", bias=None if bias_t is None else f32(bias_t),
                                           rows=r, cols=c)
    got = f32(out)[np.ix_(r, c)]
    _check(got, ref, f"m={m} n={n} k={k} {variant}", out_dtype="float16" if out_dtype == torch.float16 else "bfloat16")
    return out


def test_config1():
    _run_and_check(32, 1024, 2048, rows=32, cols=1024)


# trans_b=False (row_major): b given as (k, n); the op transposes it on the GPU, then runs the GEMM.
# Checked against the oracle on the (n, k) weight, and bit for bit against trans_b=True on b.T.
@pytest.mark.parametrize("m,n,k,mode,bias,fp16,e5", [
    (1, 2112, 7168, "K", False, False, False),     # stream kernel, split K
    (64, 1040, 2048, "MN", True, True, False),     # n not a multiple of the 64-byte transpose tile
    (300, 1536, 1024, "K", True, False, True),     # LDS kernel, e5m2
])
def test_trans_b_false(m, n, k, mode, bias, fp16, e5):
    dtype = torch.float8_e5m2 if e5 else torch.float8_e4m3fn
    say(f"gemm_a8w8 trans_b=False m={m} n={n} k={k} mode={mode} bias={bias} fp16={fp16} {_fmt(dtype)}")
    q, s, b, bs = _fp8_inputs(m, n, k, seed=m + 5, dtype=dtype)
    bias_t = torch.randn(n, device=DEV, generator=workloads.generator(m, DEV)) if bias else None
    a_scale = s.t().contiguous() if mode == "K" else s
    out_dtype = torch.float16 if fp16 else None
    b_kn = b.t().contiguous()  # (k, n)
    out = aklr_amd.gemm_a8w8_blockwise_scaled(q, b_kn, a_scale, bs, scale_major_mode=mode, trans_b=False,
                                              bias=bias_t, out_dtype=out_dtype)
    assert isinstance(out, torch.Tensor), f"not served: {out}"
    want = aklr_amd.gemm_a8w8_blockwise_scaled(q, b, a_scale, bs, scale_major_mode=mode, bias=bias_t,
                                               out_dtype=out_dtype)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16)), "trans_b=False differs from trans_b=True on b.T"
    r, c = _sample(m, n, 64, 512, m)
    ref = ogemm.gemm_a8w8_blockwise_scaled(u8(q), u8(b), s.cpu().numpy(), bs.cpu().numpy(), fmt=_fmt(dtype),
                                           scale_major_mode="MN", bias=None if bias_t is None else f32(bias_t),
                                           rows=r, cols=c)
    _check(f32(out)[np.ix_(r, c)], ref, f"trans_b=False m={m} n={n} k={k}",
           out_dtype="float16" if fp16 else "bfloat16")


def test_transpose_b8_exact():
    # the byte transpose itself, through the C ABI, on a ragged (k, n) with a padded source stride
    from aklr_amd import _lib
    L = _lib.lib()
    g = workloads.generator(3, DEV)
    rows, cols, ld = 272, 1040, 1072
    src = torch.randint(0, 256, (rows, ld), dtype=torch.uint8, device=DEV, generator=g)
    dst = torch.full((cols, rows), 7, dtype=torch.uint8, device=DEV)
    st = L.aklr_transpose_b8(src.data_ptr(), rows, cols, ld, dst.data_ptr(), rows,
                             torch.cuda.current_stream().cuda_stream)
    assert st == 0, L.aklr_status_string(st)
    torch.cuda.synchronize()
    assert torch.equal(dst, src[:, :cols].t())


@pytest.mark.parametrize("nk", workloads.DEEPSEEK_NK)
@pytest.mark.parametrize("m", workloads.DECODE_M)
def test_decode_row_major(m, nk):
    n, k = nk
    _run_and_check(m, n, k, rows=128, cols=n if n * k <= 2**25 else 1024, seed=m)


@pytest.mark.parametrize("nk", workloads.DEEPSEEK_NK)
@pytest.mark.parametrize("m", [1, 16, 128])
def test_decode_b_shuffled(m, nk):
    n, k = nk
    _run_and_check(m, n, k, variant="b_shuffled", rows=128, cols=1024, seed=m + 100)


# Stream plans whose waves split K (2 or 4 K groups of one column tile, one K split): K ranges that are
# whole multiples of the group count and ones that leave a group's last block past the range (k = 1152:
# 9 blocks over 2 groups; k = 1408: 11 over 4), 1 and 2 row tiles, ragged n, both weight layouts,
# bias and fp16 output. The plan for each is in the comment.
@pytest.mark.parametrize("m,n,k,variant,bias,fp16", [
    (1, 4096, 8192, "b_shuffled", False, False),    # 4 groups, 64 blocks
    (16, 4096, 4096, "row_major", True, False),     # 4 groups
    (5, 7168, 2048, "b_shuffled", False, True),     # 2 groups
    (32, 8192, 1024, "row_major", False, False),    # 2 groups, 2 row tiles
    (20, 4096, 2048, "b_shuffled", False, False),   # 4 groups, 2 row tiles
    (3, 8192, 1152, "row_major", False, False),     # 2 groups, 9 blocks
    (16, 4096, 1408, "b_shuffled", False, False),   # 4 groups, 11 blocks
    (9, 4112, 4096, "row_major", True, True),       # 4 groups, 257 workgroups, ragged last tile
])
def test_wave_split_k_plans(m, n, k, variant, bias, fp16):
    out = _run_and_check(m, n, k, variant=variant, bias=bias, out_dtype=torch.float16 if fp16 else None,
                         seed=m + 300, rows=64, cols=min(n, 2048))
    if m == 1:  # the groups' sums meet in a fixed order: bitwise reproducible
        again = _run_and_check(m, n, k, variant=variant, seed=m + 300, rows=8, cols=64)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), again.view(torch.int16))


# Stream plans at 4 and 8 row tiles with one column tile per wave (K <= 64 blocks, <= 256 column groups):
# both layouts, bias, fp16 output, a ragged last column group and ragged rows.
@pytest.mark.parametrize("m,n,k,variant,bias,fp16", [
    (64, 7168, 2048, "b_shuffled", False, False),
    (128, 4096, 8192, "row_major", True, False),
    (100, 4112, 4096, "b_shuffled", False, False),
    (50, 8192, 1024, "row_major", False, True),
])
def test_stream_one_column_tile_plans(m, n, k, variant, bias, fp16):
    _run_and_check(m, n, k, variant=variant, bias=bias, out_dtype=torch.float16 if fp16 else None, seed=m + 500,
                   rows=64, cols=min(n, 2048))


@pytest.mark.parametrize("nk", workloads.DEEPSEEK_NK)
@pytest.mark.parametrize("m", workloads.PREFILL_M)
def test_prefill_row_major(m, nk):
    n, k = nk
    _run_and_check(m, n, k, rows=48, cols=384, seed=m)


@pytest.mark.parametrize("nk", workloads.DEEPSEEK_NK)
def test_prefill_b_shuffled(nk):
    n, k = nk
    _run_and_check(1024, n, k, variant="b_shuffled", rows=48, cols=384, seed=3)


@pytest.mark.parametrize("m", [5, 200, 700])
def test_row_major_a_scale_shuffled_b(m):
    _run_and_check(m, 2112, 7168, variant="b_shuffled_row_major_a_scale", seed=11)


@pytest.mark.parametrize("m", [7, 40, 300, 777])
def test_mn_scales_bias_fp16(m):
    _run_and_check(m, 2112, 1536, mode="MN", bias=True, out_dtype=torch.float16, seed=21)


@pytest.mark.parametrize("m", [16, 100, 256, 640])
def test_e5m2(m):
    _run_and_check(m, 1024, 2048, dtype=torch.float8_e5m2, seed=31)


# e5m2 on the wave-split-K plan (m = 16, 4096 x 4096: 4 K groups) and on one column tile per wave at 4 row
# tiles (m = 64, 7168 x 2048)
@pytest.mark.parametrize("m,n,k", [(16, 4096, 4096), (64, 7168, 2048)])
def test_e5m2_stream_plans(m, n, k):
    _run_and_check(m, n, k, dtype=torch.float8_e5m2, seed=33, rows=64, cols=1024)


@pytest.mark.parametrize("m,n,k", [(1, 16, 128), (129, 48, 128), (17, 2112, 256), (130, 144, 384),
                                   (1, 16, 65536), (16, 256, 16384), (33, 64, 8192),
                                   (513, 2112, 256), (600, 144, 384), (1000, 48, 1024)])
def test_small_and_ragged(m, n, k):
    _run_and_check(m, n, k, seed=41)


# Stream-kernel edges (m <= 128): column groups past n (n not a multiple of the group's 64 or 128
# columns, whole waves past n), one K block, padded row tiles (m = 96 runs 8 row tiles), bias on both
# store paths (one and two column tiles per wave), and K splits with a ragged last split. The short-K
# plan of two waves and one split at 4 and 8 row tiles: 7168 x 2048 at m = 96, a ragged last 32-column
# group (6160 columns, 193 groups) with padded rows, and 256 groups at m = 50.
@pytest.mark.parametrize("m,n,k,bias", [(20, 16, 640, True), (90, 4112, 1024, True), (96, 7168, 2048, False),
                                        (128, 4096, 128, True), (33, 48, 128, False), (120, 2112, 7168, True),
                                        (65, 6144, 2304, False), (3, 4112, 1024, True), (16, 48, 384, False),
                                        (100, 6160, 1024, True), (50, 8192, 2048, False)])
def test_stream_shapes(m, n, k, bias):
    _run_and_check(m, n, k, bias=bias, seed=51)
    _run_and_check(m, n, k, variant="b_shuffled", bias=False, seed=52)


# The planner's fill plans, one per compute-wave count it picks, each with a ragged last column group
# (some of its waves' columns past n) and column groups straddling 128-column b_scale blocks (widths of
# 32, 96 and 112 columns): 1 row tile at 1, 3 and 7 waves, 4 and 8 row tiles at 2, 6 and 7 waves.
@pytest.mark.parametrize("m,n,k,bias,fp16", [
    (16, 1904, 7168, True, False),     # 1 wave x 2 tiles, 4 splits
    (4, 22960, 1024, False, True),     # 3 waves x 2 tiles
    (1, 26784, 1536, True, False),     # 7 waves x 1 tile
    (64, 1904, 4096, False, False),    # 4 row tiles, 2 waves, 4 splits
    (96, 5680, 16384, True, True),     # 8 row tiles, 6 waves
    (50, 6624, 16384, False, False),   # 4 row tiles, 7 waves
])
def test_fill_plans(m, n, k, bias, fp16):
    out_dtype = torch.float16 if fp16 else None
    _run_and_check(m, n, k, bias=bias, out_dtype=out_dtype, seed=61)
    _run_and_check(m, n, k, variant="b_shuffled", seed=62)


# The 192x192 LDS tile (planned for N = 2112 = 11 x 192 at m >= 2048): a ragged last row tile (m not a
# multiple of 192), 2 K splits at m = 2048 (121 tiles), bias and fp16 output on both variants.
@pytest.mark.parametrize("m,n,k,bias,fp16", [
    (2048, 2112, 7168, False, False),
    (4000, 2112, 7168, True, True),
    (2500, 2112, 1024, True, False),
])
def test_192_row_tiles(m, n, k, bias, fp16):
    out_dtype = torch.float16 if fp16 else None
    _run_and_check(m, n, k, bias=bias, out_dtype=out_dtype, seed=65, rows=128, cols=512)
    _run_and_check(m, n, k, variant="b_shuffled", seed=66, rows=128, cols=512)


# The 64-row LDS tiles on row-major weights (preshuffled ones take the row-block stream plans there), every
# output compared. At m = 129..256 on K <= 16 blocks: 64x128 on wide N (7168 x 2048 at m = 256 and 192; a
# ragged last column tile of 16, 200 x 4112 x 256), unsplit 64x64 up to N = 4096 (256 x 3072 x 1536;
# 130 x 3072 x 1536 with a ragged last row tile of 2 rows), 64x64 with 4 K splits (240 x 1024 x 2048).
# 64x64 at m = 65..128 on K <= 16 blocks, where the 2-wave row blocks do not fit (n > 4096): 7168 x 2048 at
# m = 128 and 96, 7168 x 1536 with bias, a ragged last column tile of 16 (80 x 4112 x 1024). Bias, fp16
# output and e5m2.
@pytest.mark.parametrize("m,n,k,bias,fp16,e5", [
    (256, 7168, 2048, False, False, False),
    (192, 7168, 2048, False, True, False),
    (256, 3072, 1536, True, True, False),
    (130, 3072, 1536, True, True, False),
    (240, 1024, 2048, True, False, True),
    (200, 4112, 256, True, False, False),
    (128, 7168, 2048, True, True, False),
    (96, 7168, 2048, False, False, True),
    (100, 7168, 1536, True, False, False),
    (80, 4112, 1024, False, True, False),
])
def test_64_row_tiles(m, n, k, bias, fp16, e5):
    assert aklr_amd._lib.lib().aklr_gemm_a8w8_blockscale_kernel(m, n, k, aklr_amd._lib.B_ROW_MAJOR) == 1
    _run_and_check(m, n, k, bias=bias, out_dtype=torch.float16 if fp16 else None, seed=m + 700,
                   dtype=torch.float8_e5m2 if e5 else torch.float8_e4m3fn, rows=m, cols=n)


# Stream plans with row blocks (preshuffled weights): 64-row blocks over the grid's z (m = 65..128 on K <= 64
# blocks; m = 129..256 on K <= 16 blocks), 32-row blocks at m = 33..64 on K <= 64 blocks. 64-column
# workgroups of 4 waves (32 columns and 2 waves at 3072 x 1536 and m <= 128; 128 columns and 8 waves at
# 7168 x 2048 and 8192 x 1024 past m = 128), K split into as many parts as keep <= 256 workgroups at >= 8
# K blocks each (3 at 2112 x 7168, the last holding 18 K blocks;
# 5 at 1536 x 7168, the last holding 8; 7 at 576 x 7168); a second block of one row (m = 65 and 33), a
# last block of 8 rows (m = 200) and of 18 (m = 50), ragged n (4112: the last group holds 16 columns),
# fp16 output, row-major weights on the 2-wave plan (3072 x 1536 at m = 64, 100 and 128, with bias; 2048 x
# 2048 at m = 64 with 2 K splits), 32-row blocks whose waves split K at 16..32 K blocks (4 groups: 512 x
# 4096 at m = 64, 1024 x 4096 at m = 128, 2048 x 2048 at m = 50, 1040 x 3072 at m = 40 with a last column
# group of 16; 2 groups: 1536 x 4096 at m = 96, 2048 x 4096 at m = 128), 64-row blocks at m = 257..1024
# on 16..32 K blocks (8 waves: 1024 x 1536 x 4096, 640 x 2048 x 2048, 1000 x 1536 x 4096 with a last block
# of 40 rows; 4 waves: 768 x 1024 x 4096), 64-row blocks of 2 K groups of 2 waves at m = 129..1024 (256 x
# 2048 and 256 x 1536 x 4096, 200 x 1536 x 3072 and 300 x 1536 x 4096 with last blocks of 8 and 44 rows,
# 1024 x 512 and 700 x 512 x 4096; 256 x 1536 x 2048 on 16 K blocks), 32-row
# blocks whose waves split K past m = 128 (4 groups: 256 x 512 x 4096, 192 x 512 x 3072; 2 groups: 512 x 512 x
# 4096, 200 x 768 x 4096 with a last block of 8 rows, 1024 x 256 x 4096, 300 x 512 x 3072; on 16-20 K
# blocks: 250 x 1024 and 512 x 512 x 2048, 300 x 768 x 2048 and 700 x 256 x 2560 with last blocks of 12
# and 28 rows; on 8-12 K blocks, 2 groups: 512 x 512, 256 x 512 and 128 x 512 x 1024, 300 x 768 and 100 x
# 1024 x 1536; 64-row blocks
# of 2 K groups on 12: 1024 x 512 and 256 x 2048 x 1536, on 8: 512 x 1024 and 700 x 640 x 1024, a last
# block of 60 rows; edges: 129 x 48 x 4096 (a last block of one row, 3 groups of 16 columns), 1024 x 16 x
# 1024 (one group), 1000 x 80 x 1536 (a last group of 16 columns, a last block of 8 rows); 257 x 2064 x
# 3072 on 64-row blocks of 4 waves, a last block of one row and a last group of 16 columns), and
# row-major weights at 32 K blocks, which keep the 8-row-tile stream plan. Every output compared.
@pytest.mark.parametrize("m,n,k,variant,bias,fp16,stream", [
    (128, 7168, 2048, "b_shuffled", False, False, True),
    (65, 3072, 1536, "b_shuffled", False, True, True),
    (100, 4096, 8192, "b_shuffled", False, False, True),
    (128, 2112, 7168, "b_shuffled", False, False, True),
    (128, 1536, 7168, "b_shuffled", False, True, True),
    (96, 576, 7168, "b_shuffled", False, False, True),
    (96, 4112, 4096, "row_major", True, False, True),
    (80, 4112, 4096, "b_shuffled", False, True, True),
    (256, 7168, 2048, "b_shuffled", False, False, True),
    (192, 7168, 2048, "b_shuffled", False, True, True),
    (200, 3072, 1536, "b_shuffled", False, False, True),
    (256, 8192, 1024, "b_shuffled", False, True, True),
    (250, 1024, 2048, "b_shuffled", False, False, True),  # 32-row blocks of 2 K groups, 16 K blocks
    (512, 512, 2048, "b_shuffled", False, True, True),
    (300, 768, 2048, "b_shuffled", False, False, True),
    (700, 256, 2560, "b_shuffled", False, False, True),
    (256, 1536, 2048, "b_shuffled", False, False, True),
    (512, 512, 1024, "b_shuffled", False, False, True),
    (256, 512, 1024, "b_shuffled", False, True, True),
    (300, 768, 1536, "b_shuffled", False, False, True),
    (1024, 512, 1536, "b_shuffled", False, False, True),
    (256, 2048, 1536, "b_shuffled", False, True, True),
    (128, 512, 1024, "b_shuffled", False, False, True),
    (100, 1024, 1536, "b_shuffled", False, True, True),
    (512, 1024, 1024, "b_shuffled", False, False, True),
    (700, 640, 1024, "b_shuffled", False, True, True),
    (129, 48, 4096, "b_shuffled", False, False, True),
    (1024, 16, 1024, "b_shuffled", False, True, True),
    (1000, 80, 1536, "b_shuffled", False, False, True),
    (257, 2064, 3072, "b_shuffled", False, False, True),
    (64, 3072, 1536, "b_shuffled", False, False, True),
    (33, 7168, 2048, "b_shuffled", False, True, True),
    (64, 2112, 7168, "b_shuffled", False, False, True),
    (50, 4112, 4096, "b_shuffled", False, False, True),
    (64, 4096, 8192, "b_shuffled", False, True, True),
    (48, 8192, 1024, "b_shuffled", False, False, True),
    (64, 3072, 1536, "row_major", True, False, True),
    (100, 3072, 1536, "row_major", False, True, True),
    (128, 3072, 1536, "row_major", True, False, True),
    (64, 2048, 2048, "row_major", False, False, True),
    (64, 512, 4096, "b_shuffled", False, False, True),
    (128, 1024, 4096, "b_shuffled", False, True, True),
    (96, 1536, 4096, "b_shuffled", False, False, True),
    (50, 2048, 2048, "b_shuffled", False, False, True),
    (128, 2048, 4096, "b_shuffled", False, False, True),
    (40, 1040, 3072, "b_shuffled", False, True, True),
    (1024, 1536, 4096, "b_shuffled", False, False, True),
    (512, 512, 4096, "b_shuffled", False, True, True),
    (1000, 1536, 4096, "b_shuffled", False, False, True),
    (640, 2048, 2048, "b_shuffled", False, False, True),
    (300, 1536, 4096, "b_shuffled", False, True, True),
    (768, 1024, 4096, "b_shuffled", False, False, True),
    (256, 512, 4096, "b_shuffled", False, False, True),
    (192, 512, 3072, "b_shuffled", False, True, True),
    (200, 768, 4096, "b_shuffled", False, False, True),
    (1024, 256, 4096, "b_shuffled", False, True, True),
    (300, 512, 3072, "b_shuffled", False, False, True),
    (256, 2048, 4096, "b_shuffled", False, True, True),
    (256, 1536, 4096, "b_shuffled", False, False, True),
    (200, 1536, 3072, "b_shuffled", False, False, True),
    (1024, 512, 4096, "b_shuffled", False, True, True),
    (700, 512, 4096, "b_shuffled", False, False, True),
])
def test_row_block_plans(m, n, k, variant, bias, fp16, stream):
    layout = aklr_amd._lib.B_ROW_MAJOR if variant == "row_major" else aklr_amd._lib.B_PRESHUFFLE_16x16
    assert aklr_amd._lib.lib().aklr_gemm_a8w8_blockscale_kernel(m, n, k, layout) == (0 if stream else 1)
    _run_and_check(m, n, k, variant=variant, bias=bias, out_dtype=torch.float16 if fp16 else None, seed=m + 800,
                   rows=m, cols=n)


# LDS plans of 64-row tiles where the output is small: 64x64 tiles at 4, 2 and 1 K splits (256 x 512 x
# 5120, 512 x 1024 x 4096 / 1000 x 512 x 4096 / 777 x 1024 x 4096 and 384 x 2048 x 3072), 64x128 unsplit
# (512 x 4096 x 1024; 300 x 4112 x 2048 with a ragged last row tile of 44 rows and a last column tile of
# 16) and with 3 and 4 K splits (2112 x 7168 at m = 256, 200 and 192: last column tiles of 64, and at
# m = 200 a last row tile of 8); on 2-4 K blocks at a row pitch of 8 KiB (1024 x 4096 x 512, 2048 x 4096 x
# 256), whose output stores are non-temporal; both layouts, bias, fp16 and e5m2. Every output compared.
@pytest.mark.parametrize("m,n,k,variant,bias,fp16,e5", [
    (256, 512, 5120, "b_shuffled", False, False, False),
    (512, 1024, 4096, "row_major", True, True, False),
    (1000, 512, 4096, "row_major", False, False, False),
    (777, 1024, 4096, "row_major", False, False, True),
    (384, 2048, 3072, "row_major", False, True, False),
    (512, 4096, 1024, "b_shuffled", False, False, False),
    (300, 4112, 2048, "row_major", True, False, False),
    (256, 2112, 7168, "b_shuffled", False, False, False),
    (192, 2112, 7168, "b_shuffled", False, True, False),
    (200, 2112, 7168, "row_major", True, False, False),
    (1024, 4096, 512, "b_shuffled", False, False, False),
    (2048, 4096, 256, "row_major", True, True, False),
])
def test_small_output_lds_plans(m, n, k, variant, bias, fp16, e5):
    layout = aklr_amd._lib.B_ROW_MAJOR if variant == "row_major" else aklr_amd._lib.B_PRESHUFFLE_16x16
    assert aklr_amd._lib.lib().aklr_gemm_a8w8_blockscale_kernel(m, n, k, layout) == 1
    _run_and_check(m, n, k, variant=variant, bias=bias, out_dtype=torch.float16 if fp16 else None,
                   dtype=torch.float8_e5m2 if e5 else torch.float8_e4m3fn, seed=m + 900, rows=m, cols=n)


# A K-major a_scale against a column-major one: the same scale values in the same fold order, so bitwise
# the same outputs; preshuffled weights (K-major a_scale marked is_row_major) and row-major weights
# (scale_major_mode K against MN). Preshuffled: the LDS kernel's ring of 16-row x 4-block a_scale
# quarters (64x64, 64x128, 128x128 and 128x192 tiles, 1-4 K splits, K ranges of 8-32 blocks and of 14
# at 7168 / 4 splits, whose last group is part empty; 1500 rows: a ragged last row tile) and its
# per-stage loads (128x256, 192x192 and 256x256 tiles), the stream kernel's ring on
# 64-row blocks of 24-32 K blocks (1024 x 1024 x 4096 on 4 waves, 1024 x 1536 x 4096 and 1000 x 1536 x
# 4096 on 8, a ragged last row block of 40 rows; 300 x 4112 x 2048, 16 K blocks, takes the per-stage
# loads), and per-stage loads on the blocks whose waves split K (32-row: 64 x 512 and 128 x 1024 x 4096 in
# 4 K groups, 100 x 1040 x 3072 in 2 over 24 K blocks, ragged rows and columns; 64-row: 1000 x 512 x 4096
# and 600 x 768 x 3072, ragged last blocks of 40 and 24 rows).
@pytest.mark.parametrize("m,n,k", [(256, 512, 5120), (1000, 512, 4096), (512, 4096, 1024), (1024, 1024, 4096),
                                   (300, 4112, 2048), (1024, 1536, 4096), (256, 2112, 7168), (1024, 4096, 4096),
                                   (64, 512, 4096), (128, 1024, 4096), (100, 1040, 3072), (600, 768, 3072),
                                   (1000, 1536, 4096),
                                   (1500, 512, 3584), (2048, 1024, 4096), (4096, 512, 4096), (2048, 1536, 4096),
                                   (2048, 2112, 7168), (1100, 7168, 2048), (1100, 24576, 1536)])
def test_k_major_a_scale_bitwise(m, n, k):
    say(f"gemm_a8w8 K-major a_scale m={m} n={n} k={k}")
    q, s, b, bs = _fp8_inputs(m, n, k, m + 950, torch.float8_e4m3fn)  # s: [k / 128, m] group-major
    bb = layouts.shuffle_weight(b)
    out_cm = aklr_amd.gemm_a8w8_blockwise_scaled(q, bb, s.view(m, k // 128), bs, operand_format="none:preshuffled")
    sk = s.t().contiguous()
    sk.is_row_major = True
    out_km = aklr_amd.gemm_a8w8_blockwise_scaled(q, bb, sk, bs, operand_format="none:preshuffled")
    assert torch.equal(out_cm.view(torch.int16), out_km.view(torch.int16)), "preshuffled: K-major a_scale differs"
    out_rk = aklr_amd.gemm_a8w8_blockwise_scaled(q, b, s.t().contiguous(), bs)
    out_rmn = aklr_amd.gemm_a8w8_blockwise_scaled(q, b, s, bs, scale_major_mode="MN")
    assert torch.equal(out_rk.view(torch.int16), out_rmn.view(torch.int16)), "row-major: K-major a_scale differs"
    r, c = _sample(m, n, 64, 512, seed=m)
    ref = ogemm.gemm_a8w8_blockwise_scaled(u8(q), u8(b), s.cpu().numpy(), bs.cpu().numpy(), scale_major_mode="MN",
                                           rows=r, cols=c)
    got = f32(out_km)[np.ix_(r, c)]
    assert ogemm.within_north_star(got, ref) and ogemm.within_contract_tolerance(got, ref)


# The long-K plan (one row tile, >= 96 K blocks, 192-256 workgroups of 32 columns, one K split, each
# workgroup starting its K walk at its own block): a ragged last workgroup (n = 6160: its second column
# tile past n) at a K range that 193 workgroups do not divide, 256 workgroups at 100 K blocks, MN scales,
# bias, fp16 and e5m2. The fused entry runs the two kernels there and equals the two ops bit for bit.
@pytest.mark.parametrize("m,n,k,mode,bias,fp16,e5", [
    (13, 6160, 12288, "K", True, True, False),
    (1, 8192, 12800, "MN", False, False, False),
    (16, 7168, 16384, "K", False, False, True),
    (5, 7168, 16384, "MN", True, False, False),
])
def test_long_k_plan(m, n, k, mode, bias, fp16, e5):
    assert aklr_amd._lib.lib().aklr_gemm_a8w8_blockscale_workspace_bytes(m, n, k) == 0, "expected one K split"
    dtype = torch.float8_e5m2 if e5 else torch.float8_e4m3fn
    out_dtype = torch.float16 if fp16 else None
    _run_and_check(m, n, k, mode=mode, bias=bias, out_dtype=out_dtype, dtype=dtype, seed=63, cols=1024)
    if not e5:
        _run_and_check(m, n, k, variant="b_shuffled", seed=64, cols=1024)
        assert aklr_amd._lib.lib().aklr_quant_gemm_a8w8_blockscale_fused(m, n, k) == 0


# 192- and 224-column LDS tiles (planned where they divide N): ragged row tiles, bias and fp16 output on
# the odd last column tile's 8-byte stores, b_scale blocks straddled by a wave's columns (tiles start at
# multiples of 64 or 32 columns), 256- and 128-row tiles, the 4 x 2 wave layout and the uneven B slabs
# of the 224-column tile.
@pytest.mark.parametrize("m,n,k,bias,fp16", [(2500, 2112, 1536, True, True), (4000, 2112, 512, True, False),
                                             (4100, 4032, 1024, False, True), (2000, 7168, 2048, True, True),
                                             (3000, 4480, 1024, False, False)])
def test_192_224_column_tiles(m, n, k, bias, fp16):
    _run_and_check(m, n, k, mode="MN", bias=bias, out_dtype=torch.float16 if fp16 else None, seed=61)
    _run_and_check(m, n, k, variant="b_shuffled", bias=False, seed=62)


# Fused per-1x128 quantization + GEMM: equal bit for bit to per_group_quant_fp8 then
# gemm_a8w8_blockwise_scaled, on the fused stream kernel (m <= 16: one row tile, one and two column
# tiles per wave, K splits, ragged rows and columns, an x row stride past k) and on the two-kernel
# path beyond (m = 20 .. 300).
@pytest.mark.parametrize("m,n,k,shuffled,bias,fp16", [
    (1, 7168, 16384, True, False, False), (16, 7168, 16384, True, False, False), (4, 2112, 7168, True, False, False),
    (16, 24576, 1536, True, False, False), (13, 4112, 1024, False, True, True), (64, 7168, 2048, True, False, False),
    (7, 48, 384, False, True, False), (20, 2112, 128, False, False, True), (100, 2112, 7168, True, False, False),
    (300, 1024, 2048, False, True, False), (1, 4096, 8192, True, False, False)])
def test_quant_gemm_fused_matches_two_ops(m, n, k, shuffled, bias, fp16):
    say(f"quant_gemm_a8w8 m={m} n={n} k={k} shuffled={shuffled} bias={bias} fp16={fp16}")
    wide = workloads.activations(m, k + 64, seed=71, device=DEV)
    x = wide[:, 32:32 + k]  # row stride k + 64, 64-byte aligned start
    b, bs = workloads.blockwise_fp8_weight(n, k, seed=72, device=DEV)
    bias_t = torch.randn(n, device=DEV, generator=workloads.generator(73, DEV)) if bias else None
    od = torch.float16 if fp16 else None
    q, s = aklr_amd.per_group_quant_fp8(x.contiguous())
    if shuffled:
        bb = layouts.shuffle_weight(b)
        ref = aklr_amd.gemm_a8w8_blockwise_scaled(q, bb, s.view(m, k // 128), bs, bias=bias_t, out_dtype=od,
                                                  operand_format="none:preshuffled") if bias_t is None else None
        if ref is None:  # the shuffled op variant takes no bias: compare against the row-major op
            ref = aklr_amd.gemm_a8w8_blockwise_scaled(q, b, s.t().contiguous(), bs, bias=bias_t, out_dtype=od)
        got = aklr_amd.quant_gemm_a8w8_blockwise_scaled(x, bb, bs, bias=bias_t, out_dtype=od,
                                                        operand_format="none:preshuffled")
    else:
        ref = aklr_amd.gemm_a8w8_blockwise_scaled(q, b, s.t().contiguous(), bs, bias=bias_t, out_dtype=od)
        got = aklr_amd.quant_gemm_a8w8_blockwise_scaled(x, b, bs, bias=bias_t, out_dtype=od)
    assert isinstance(got, torch.Tensor) and isinstance(ref, torch.Tensor), (got, ref)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), \
        f"fused quant+GEMM differs from the two ops: max|diff| {(got.float() - ref.float()).abs().max().item():.3e}"
    info = aklr_amd.quant_gemm_a8w8_blockwise_scaled.serving(x, b if not shuffled else bb, bs, bias=bias_t,
                                                              out_dtype=od,
                                                              operand_format="none:preshuffled" if shuffled else "none:none")
    # one launch at m <= 16 on the DeepSeek-V3 shapes of up to 56 K blocks; elsewhere the library's plan
    # decides (a GEMM plan that splits K over its waves, e.g. 4096 x 8192 or 4112 x 1024, or the long-K
    # plan of 7168 x 16384, runs the two kernels)
    fused = aklr_amd._lib.lib().aklr_quant_gemm_a8w8_blockscale_fused(m, n, k) == 1
    if m <= 16 and (n, k) in workloads.DEEPSEEK_NK:
        assert fused == ((n, k) != (7168, 16384))
    assert info.kernel_ref.endswith(":stream_fused" if fused else (":stream" if m <= 128 else ":lds"))


def test_quant_gemm_into_strided_out():
    # out= through the op (contiguous, as its contract takes it), then a column slice of a wider buffer
    # through the C ABI's row stride: the fused path (m = 4) and the two-kernel path (m = 40); the columns
    # around the slice stay untouched
    L = aklr_amd._lib.lib()
    for m in (4, 40):
        n, k = 2112, 7168
        x = workloads.activations(m, k, seed=81, device=DEV)
        b, bs = workloads.blockwise_fp8_weight(n, k, seed=82, device=DEV)
        bb = layouts.shuffle_weight(b)
        q, s = aklr_amd.per_group_quant_fp8(x)
        ref = aklr_amd.gemm_a8w8_blockwise_scaled(q, bb, s.view(m, k // 128), bs, operand_format="none:preshuffled")
        out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
        got = aklr_amd.quant_gemm_a8w8_blockwise_scaled(x, bb, bs, out=out, operand_format="none:preshuffled")
        assert got is out
        wide = torch.full((m, n + 64), float("nan"), dtype=torch.bfloat16, device=DEV)
        ws_bytes = L.aklr_quant_gemm_a8w8_blockscale_workspace_bytes(m, n, k)
        ws = torch.zeros(max(ws_bytes, 16), dtype=torch.uint8, device=DEV)
        st = L.aklr_quant_gemm_a8w8_blockscale(x.data_ptr(), k, bb.data_ptr(), k, bs.data_ptr(), bs.stride(0), None,
                                               wide[:, 32:].data_ptr(), n + 64, m, n, k, aklr_amd._lib.B_PRESHUFFLE_16x16,
                                               0, ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
        assert st == 0
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
        assert torch.equal(wide[:, 32:32 + n].view(torch.int16), ref.view(torch.int16))
        assert torch.isnan(wide[:, :32].float()).all() and torch.isnan(wide[:, 32 + n:].float()).all()


def test_out_buffer_and_determinism():
    m, n, k = 64, 7168, 16384
    q, s, b, bs = _fp8_inputs(m, n, k, seed=5)
    out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    r1 = aklr_amd.gemm_a8w8_blockwise_scaled(q, b, s.t().contiguous(), bs, out=out)
    assert r1 is out
    r2 = aklr_amd.gemm_a8w8_blockwise_scaled(q, b, s.t().contiguous(), bs)
    torch.cuda.synchronize()
    assert not torch.isnan(out.float()).any()
    assert torch.equal(r1.view(torch.int16), r2.view(torch.int16)), "decode GEMM is not bitwise reproducible"


def test_scale_linearity():
    # doubling every b_scale doubles the output exactly (power-of-two scaling is exact in fp32)
    m, n, k = 2048, 2112, 1536
    q, s, b, bs = _fp8_inputs(m, n, k, seed=6)
    o1 = aklr_amd.gemm_a8w8_blockwise_scaled(q, b, s.t().contiguous(), bs).float()
    o2 = aklr_amd.gemm_a8w8_blockwise_scaled(q, b, s.t().contiguous(), bs * 2).float()
    torch.cuda.synchronize()
    assert torch.equal(o1 * 2, o2)


# ---------------------------------------------------------------------------------------------
# MXFP4
def _mxfp4_run(m, n, k, shuffled, seed=0, rows=64, cols=512, bias=False):
    say(f"gemm_a4w4_mxfp4 m={m} n={n} k={k} shuffled={shuffled} bias={bias}")
    x = workloads.activations(m, k, seed=seed, device=DEV)
    qa, sa = aklr_amd.dynamic_mxfp4_quant(x, shuffle=shuffled)
    qa_rm, sa_rm = aklr_amd.dynamic_mxfp4_quant(x, shuffle=False)
    wb, sb = workloads.mxfp4_weight(n, k, seed=seed + 1, device=DEV)
    bias_t = torch.randn(n, device=DEV, generator=workloads.generator(seed + 9, DEV)) if bias else None
    if shuffled:
        out = aklr_amd.gemm_a4w4_mxfp4(qa, layouts.shuffle_weight(wb), sa, layouts.e8m0_scales(sb), bias=bias_t)
    else:
        out = aklr_amd.gemm_a4w4_mxfp4(qa, wb, sa, sb, bias=bias_t, operand_format="none:none")
    assert isinstance(out, torch.Tensor), f"not served: {out}"
    torch.cuda.synchronize()
    r, c = _sample(m, n, rows, cols, seed)
    ref = ogemm.gemm_a4w4_mxfp4(u8(qa_rm), u8(wb), u8(sa_rm), u8(sb), bias=None if bias_t is None else f32(bias_t),
                                rows=r, cols=c)
    got = f32(out)[np.ix_(r, c)]
    _check(got, ref, f"mxfp4 m={m} n={n} k={k}", contract=False)
    # the contract's own bound, DotProductBound(max_split_k=1) (aklr/ops/gemm/contract.py:375): M is the
    # product of the operands' absolute values (sign bits cleared, as the reference's absolute_value does)
    mag = ogemm.gemm_a4w4_mxfp4(u8(qa_rm) & 0x77, u8(wb) & 0x77, u8(sa_rm), u8(sb),
                                bias=None if bias_t is None else np.abs(f32(bias_t)), rows=r, cols=c)
    peak = float(np.max(np.abs(got - ref) / ogemm.dot_product_bound(ref, mag, k)))
    say(f"  DotProductBound peak multiple {peak:.3f}")
    assert ogemm.within_dot_product_bound(got, ref, mag, k), f"mxfp4 m={m} n={n} k={k}: DotProductBound exceeded"
    return out


@pytest.mark.parametrize("shuffled", [True, False])
@pytest.mark.parametrize("nk", workloads.LLAMA70B_NK)
@pytest.mark.parametrize("m", workloads.MXFP4_M)
def test_mxfp4_llama(m, nk, shuffled):
    n, k = nk
    _mxfp4_run(m, n, k, shuffled, seed=m)


@pytest.mark.parametrize("m,n,k", [(1, 16, 64), (3, 32, 192), (33, 48, 320), (200, 272, 64), (40, 160, 4160),
                                   (33, 48, 256), (129, 16, 512), (300, 272, 1024), (700, 400, 2048),
                                   (2100, 1040, 768), (1, 160, 16448), (7, 48, 20032), (20, 48, 320),
                                   (32, 160, 4160), (25, 4112, 1024), (32, 40960, 512)])
def test_mxfp4_small_and_ragged_k(m, n, k):
    _mxfp4_run(m, n, k, shuffled=True, seed=m, bias=True)
    _mxfp4_run(m, n, k, shuffled=False, seed=m + 1)


@pytest.mark.parametrize("m,n,k", [(100, 272, 512), (1500, 160, 1024), (40, 2048, 8192)])
def test_mxfp4_lds_split_k_and_determinism(m, n, k):
    # shapes whose LDS plan splits K (few 128x128 tiles, long K): results equal the oracle and repeat bitwise
    out1 = _mxfp4_run(m, n, k, shuffled=True, seed=m + 3)
    out2 = _mxfp4_run(m, n, k, shuffled=True, seed=m + 3)
    torch.cuda.synchronize()
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16))


def test_quant_gemm_pipeline_matches_oracle_end_to_end():
    # the oracle quantizes too: activations -> codes/scales -> GEMM, all from the same bf16 input
    m, n, k = 16, 2112, 7168
    x = workloads.activations(m, k, seed=77, device=DEV)
    b, bs = workloads.blockwise_fp8_weight(n, k, seed=78, device=DEV)
    q, s = aklr_amd.per_group_quant_fp8(x)
    out = aklr_amd.gemm_a8w8_blockwise_scaled(q, layouts.shuffle_weight(b), s.view(m, k // 128), bs,
                                              operand_format="none:preshuffled")
    torch.cuda.synchronize()
    q_ref, s_ref = oquant.per_group_quant_fp8(bf16_bits(x))
    ref = ogemm.gemm_a8w8_blockwise_scaled(q_ref, u8(b), s_ref, bs.cpu().numpy(), scale_major_mode="MN")
    _check(out, ref, "pipeline")


def test_workspace_shared_across_shapes():
    # one stream's split-K workspace serves calls of different plans in any order: a call with few
    # column groups and many splits, then one with many column groups, then the first again
    shapes = [(1, 2112, 7168), (1, 24576, 1536), (16, 7168, 16384), (1, 2112, 7168), (128, 2112, 7168),
              (1, 24576, 1536)]
    for i, (m, n, k) in enumerate(shapes):
        _run_and_check(m, n, k, variant="b_shuffled", rows=128, cols=2048, seed=60 + i)


@pytest.mark.parametrize("nk", workloads.DEEPSEEK_NK)
@pytest.mark.parametrize("m", workloads.DECODE_M)
def test_quant_gemm_fused_against_the_oracle(m, nk):
    # quant_gemm_a8w8_blockwise_scaled (one launch at m <= 16) straight against the oracle, which quantizes
    # the same bf16 input itself (aklr/ops/quant/reference.py:9-28, then aklr/ops/gemm/reference.py:90-105)
    n, k = nk
    say(f"quant_gemm vs oracle m={m} n={n} k={k}")
    x = workloads.activations(m, k, seed=90 + m, device=DEV)
    b, bs = workloads.blockwise_fp8_weight(n, k, seed=91, device=DEV)
    out = aklr_amd.quant_gemm_a8w8_blockwise_scaled(x, layouts.shuffle_weight(b), bs, operand_format="none:preshuffled")
    assert isinstance(out, torch.Tensor), out
    torch.cuda.synchronize()
    r, c = _sample(m, n, 128, 1024, seed=m)
    q_ref, s_ref = oquant.per_group_quant_fp8(bf16_bits(x))
    ref = ogemm.gemm_a8w8_blockwise_scaled(q_ref, u8(b), s_ref, bs.cpu().numpy(), scale_major_mode="MN", rows=r, cols=c)
    _check(f32(out)[np.ix_(r, c)], ref, f"quant_gemm m={m} n={n} k={k}")

"""GPU check that a finished split-K call leaves no tagged arrival word behind.

Each split output tile's arrival word holds (launch tag, count) while its workgroups arrive; the one
that completes the count writes the reserved word 0, which no launch tag equals (tags have bit 63
set). So after a call every word of the 128 KiB counter region is either untouched or 0, and a later
launch whose tag repeats an earlier one (a HIP queue made again at the same address restarts its
dispatch ids) cannot find its count already advanced. The workspace starts as 0xFF bytes here, so the
words a plan used read 0 afterwards and the others still read all ones; a second call on the same
buffer must leave it the same way and give the same output. Covered: the FP8 stream, LDS and
fused-quantization kernels and the MXFP4 skinny, stream and LDS kernels, all on plans that split K.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import aklr_amd
from aklr_amd import _lib, layouts, workloads
from tests.helpers import say

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
WORDS = 131072 // 8
ALL_ONES = np.uint64(0xFFFFFFFFFFFFFFFF)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _check_words(ws: torch.Tensor, what: str) -> int:
    torch.cuda.synchronize()
    w = ws[:131072].cpu().numpy().view(np.uint64)
    used = int((w == 0).sum())
    bad = int(((w != 0) & (w != ALL_ONES)).sum())
    assert bad == 0, f"{what}: {bad} arrival words still hold a launch's tag"
    assert used > 0, f"{what}: no arrival word was used (the plan does not split K)"
    return used


def _twice(call, need, what):
    ws = torch.full((max(need, 131072),), 0xFF, dtype=torch.uint8, device=DEV)
    out1 = call(ws)
    used1 = _check_words(ws, what + " call 0")
    out2 = call(ws)
    used2 = _check_words(ws, what + " call 1")
    assert used1 == used2, f"{what}: the two calls used {used1} and {used2} words"
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16)), f"{what}: outputs differ"


@pytest.mark.parametrize("m,n,k", [(16, 4096, 16384), (128, 2112, 7168), (256, 2112, 7168),
                                   (100, 4096, 8192), (96, 576, 7168), (128, 1536, 7168),
                                   (64, 2112, 7168), (50, 4096, 8192),
                                   (256, 512, 5120), (1000, 512, 8192), (300, 1024, 7168)])
def test_fp8_split_words_reset(m, n, k):
    L = _lib.lib()
    need = L.aklr_gemm_a8w8_blockscale_workspace_bytes(m, n, k)
    assert need > 131072, f"({m}, {n}, {k}) is expected to split K"
    say(f"fp8 split words m={m} n={n} k={k}")
    x = workloads.activations(m, k, seed=m + 30, device=DEV)
    q, s = aklr_amd.per_group_quant_fp8(x)
    b, bs = workloads.blockwise_fp8_weight(n, k, seed=m + 31, device=DEV)
    bb = layouts.shuffle_weight(b)

    def call(ws):
        out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
        st = L.aklr_gemm_a8w8_blockscale(q.data_ptr(), k, bb.data_ptr(), k, s.data_ptr(), 1, m, bs.data_ptr(),
                                         bs.stride(0), None, out.data_ptr(), n, m, n, k, _lib.FP8_E4M3FN,
                                         _lib.B_PRESHUFFLE_16x16, _lib.OUT_BF16, ws.data_ptr(), ws.numel(), _stream())
        assert st == 0, L.aklr_status_string(st)
        return out

    _twice(call, need, f"fp8 ({m}, {n}, {k})")


def test_fused_quant_split_words_reset():
    L = _lib.lib()
    m, n, k = 16, 4096, 16384
    assert L.aklr_quant_gemm_a8w8_blockscale_fused(m, n, k) == 1
    need = L.aklr_quant_gemm_a8w8_blockscale_workspace_bytes(m, n, k)
    say(f"fused quant split words m={m} n={n} k={k}")
    x = workloads.activations(m, k, seed=40, device=DEV)
    b, bs = workloads.blockwise_fp8_weight(n, k, seed=41, device=DEV)
    bb = layouts.shuffle_weight(b)

    def call(ws):
        out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
        st = L.aklr_quant_gemm_a8w8_blockscale(x.data_ptr(), k, bb.data_ptr(), k, bs.data_ptr(), bs.stride(0), None,
                                               out.data_ptr(), n, m, n, k, _lib.B_PRESHUFFLE_16x16, _lib.OUT_BF16,
                                               ws.data_ptr(), ws.numel(), _stream())
        assert st == 0, L.aklr_status_string(st)
        return out

    _twice(call, need, "fused quant")


@pytest.mark.parametrize("m,n,k", [(1, 2048, 8192), (32, 10240, 8192), (100, 272, 4096)])
def test_mxfp4_split_words_reset(m, n, k):
    L = _lib.lib()
    need = L.aklr_gemm_a4w4_mxfp4_workspace_bytes(m, n, k)
    assert need > 131072, f"({m}, {n}, {k}) is expected to split K"
    say(f"mxfp4 split words m={m} n={n} k={k}")
    x = workloads.activations(m, k, seed=m + 50, device=DEV)
    qa, sa = aklr_amd.dynamic_mxfp4_quant(x, shuffle=True)
    wb, sb = workloads.mxfp4_weight(n, k, seed=m + 51, device=DEV)
    a8, b8 = qa.view(torch.uint8), layouts.shuffle_weight(wb).view(torch.uint8)
    sa8, sb8 = sa.view(torch.uint8), layouts.e8m0_scales(sb).view(torch.uint8)

    def call(ws):
        out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
        st = L.aklr_gemm_a4w4_mxfp4(a8.data_ptr(), k // 2, b8.data_ptr(), k // 2, sa8.data_ptr(), sa8.stride(0),
                                    sb8.data_ptr(), sb8.stride(0), None, out.data_ptr(), n, m, n, k,
                                    _lib.B_PRESHUFFLE_16x16, _lib.SCALES_SHUFFLED, _lib.OUT_BF16, ws.data_ptr(),
                                    ws.numel(), _stream())
        assert st == 0, L.aklr_status_string(st)
        return out

    _twice(call, need, f"mxfp4 ({m}, {n}, {k})")

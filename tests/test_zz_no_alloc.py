"""The no-allocation FP8 GEMM entry point against the regular one, through the C ABI.

aklr_gemm_a8w8_blockscale_noalloc runs the same kernels and plans as aklr_gemm_a8w8_blockscale with its
split-K scratch in the library's per-GPU device array, so its outputs must equal the regular entry
point's bit for bit: on two calls in a row, the second with a smaller input (the array then holds the
first call's words and partials), on plans that split K (stream and LDS kernels) and one that does not.
(That every plan fits the array is checked on the CPU, in tests/test_abi.py.)
"""
from __future__ import annotations

import pytest
import torch

import aklr_amd
from aklr_amd import _lib, layouts, workloads
from tests.helpers import say

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _inputs(m, n, k, seed):
    x = workloads.activations(m, k, seed=seed, device=DEV)
    q, s = aklr_amd.per_group_quant_fp8(x)  # s: [k/128, m], column-major a_scale
    b, bs = workloads.blockwise_fp8_weight(n, k, seed=seed + 1, device=DEV)
    return q, s, layouts.shuffle_weight(b), bs


def _call(fn, m, n, k, q, s, bb, bs, *ws):
    out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    st = fn(q.data_ptr(), k, bb.data_ptr(), k, s.data_ptr(), 1, m, bs.data_ptr(), bs.stride(0), None, out.data_ptr(),
            n, m, n, k, _lib.FP8_E4M3FN, _lib.B_PRESHUFFLE_16x16, _lib.OUT_BF16, *ws,
            torch.cuda.current_stream().cuda_stream)
    return st, out


# (first call, second smaller call): stream split plans, an LDS split plan after a stream one, and an
# unsplit LDS plan (no scratch) followed by a split stream plan
PAIRS = [((16, 4096, 16384), (4, 2112, 7168)), ((256, 2112, 7168), (128, 2112, 7168)),
         ((2048, 7168, 2048), (64, 7168, 2048))]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_regular_entry(first, second):
    L = _lib.lib()
    for i, (m, n, k) in enumerate((first, second)):
        say(f"noalloc gemm call {i}: m={m} n={n} k={k}")
        need = L.aklr_gemm_a8w8_blockscale_workspace_bytes(m, n, k)
        assert need <= _lib.NOALLOC_SCRATCH_BYTES
        q, s, bb, bs = _inputs(m, n, k, seed=10 * i + m)
        ws = torch.empty(max(need, 16), dtype=torch.uint8, device=DEV)
        st, want = _call(L.aklr_gemm_a8w8_blockscale, m, n, k, q, s, bb, bs, ws.data_ptr(), need)
        assert st == 0, L.aklr_status_string(st)
        st, got = _call(L.aklr_gemm_a8w8_blockscale_noalloc, m, n, k, q, s, bb, bs)
        assert st == 0, L.aklr_status_string(st)
        torch.cuda.synchronize()
        assert not torch.isnan(got.float()).any(), "no-allocation call left outputs unwritten"
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"call {i}: outputs differ"

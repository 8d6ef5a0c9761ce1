"""The packaged AKLR kernels (aklr_amd.schema) run as an unmodified AKLR runs them.

Each library is built from a schema's sources by AKLR's HIP build recipe (aklr_amd.schema.build, run
by __graft_entry__.build() on the CPU). Each test:

- loads it with torch.ops.load_library;
- checks its registered op the way AKLR's HipBuilder does (builder.py:309-323);
- calls it as ``run(**call)`` with the contract's call keys, writing into preallocated outputs.

Bound, written here: the outputs equal this library's own op's bit for bit. The same kernels run
behind another entry, and every kernel here is bitwise reproducible; the ops themselves are pinned
against the oracle in the other GPU tests.
"""
from __future__ import annotations

import pytest
import torch

import aklr_amd
from aklr_amd import layouts, workloads
from aklr_amd.schema import CONTRACTS, build
from tests.helpers import say

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _op(contract_id: str, variant: str):
    op = build.load(build.tested_kernel(contract_id, variant))
    c = CONTRACTS[contract_id]
    assert build.op_schema_errors(op.default._schema, c.call_keys, c.mutable) == []
    return op


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    return a.shape == b.shape and a.dtype == b.dtype and torch.equal(a.view(torch.uint8), b.view(torch.uint8))


@pytest.mark.parametrize("t,h", [(1, 7168), (300, 2048), (2048, 7168)])
def test_per_group_quant_fp8_package(t, h):
    say(f"schema per_group_quant_fp8 t={t} h={h}")
    op = _op("per_group_quant_fp8@1.0", "row_major")
    x = workloads.activations(t, h, seed=t, device=DEV)
    q = torch.empty((t, h), dtype=torch.float8_e4m3fn, device=DEV)
    s = torch.empty((h // 128, t), dtype=torch.float32, device=DEV)
    op(x=x, quantized=q, scales=s)
    q_ref, s_ref = aklr_amd.per_group_quant_fp8(x)
    torch.cuda.synchronize()
    assert _same(q, q_ref) and _same(s, s_ref)


@pytest.mark.parametrize("t,h", [(3, 7168), (1792, 7168)])
def test_per_group_quant_mxfp8_package(t, h):
    say(f"schema per_group_quant_mxfp8 t={t} h={h}")
    op = _op("per_group_quant_mxfp8@1.0", "row_major")
    x = workloads.activations(t, h, seed=t + 1, device=DEV)
    q = torch.empty((t, h), dtype=torch.float8_e4m3fn, device=DEV)
    s = torch.empty((t, h // 32), dtype=torch.uint8, device=DEV)
    op(x=x, quantized=q, scales=s)
    q_ref, s_ref = aklr_amd.per_group_quant_mxfp8(x)
    torch.cuda.synchronize()
    assert _same(q, q_ref) and _same(s, s_ref)


def _fp8_operands(m, n, k, seed):
    x = workloads.activations(m, k, seed=seed, device=DEV)
    q, s = aklr_amd.per_group_quant_fp8(x)
    b, bs = workloads.blockwise_fp8_weight(n, k, seed=seed + 1, device=DEV)
    return q, s, b, bs


# m = 4 and 16 split K over workgroups (the per-call scratch); m = 300 runs the LDS kernel
@pytest.mark.parametrize("m,n,k", [(4, 2112, 7168), (16, 7168, 2048), (300, 1536, 1024)])
def test_gemm_a8w8_b_shuffled_package(m, n, k):
    say(f"schema gemm_a8w8 b_shuffled m={m} n={n} k={k}")
    op = _op("gemm_a8w8_blockwise_scaled@1.0", "b_shuffled")
    q, s, b, bs = _fp8_operands(m, n, k, seed=m)
    bb = layouts.shuffle_weight(b)
    a_scale = s.view(m, k // 128)  # ColumnMajor storage: the transpose's bytes in a_scale's shape
    out = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    for _ in range(2):  # the second call's scratch holds the first call's words
        op(a=q, b=bb, a_scale=a_scale, b_scale=bs, scale_major_mode="K", trans_b=True,
           operand_format="none:preshuffled", bias=None, out_dtype=None, out=out)
        ref = aklr_amd.gemm_a8w8_blockwise_scaled(q, bb, a_scale, bs, operand_format="none:preshuffled")
        torch.cuda.synchronize()
        assert _same(out, ref)


@pytest.mark.parametrize("mode", ["K", "MN"])
@pytest.mark.parametrize("m,n,k", [(8, 4096, 1536), (512, 2048, 2048)])
def test_gemm_a8w8_row_major_package(mode, m, n, k):
    say(f"schema gemm_a8w8 row_major {mode} m={m} n={n} k={k}")
    op = _op("gemm_a8w8_blockwise_scaled@1.0", "row_major")
    q, s, b, bs = _fp8_operands(m, n, k, seed=m + 7)
    a_scale = s.t().contiguous() if mode == "K" else s  # (m, k/128) K-major, or (k/128, m) MN-major
    bias = torch.randn(n, device=DEV, generator=workloads.generator(m, DEV))
    out = torch.empty((m, n), dtype=torch.float16, device=DEV)
    op(a=q, b=b, a_scale=a_scale, b_scale=bs, scale_major_mode=mode, trans_b=True, operand_format="none:none",
       bias=bias, out_dtype=torch.float16, out=out)
    ref = aklr_amd.gemm_a8w8_blockwise_scaled(q, b, a_scale, bs, scale_major_mode=mode, bias=bias,
                                              out_dtype=torch.float16)
    torch.cuda.synchronize()
    assert _same(out, ref)


@pytest.mark.parametrize("m,n,k", [(8, 4096, 1536), (512, 2048, 2048)])
def test_gemm_a8w8_row_major_package_b_kn(m, n, k):
    # trans_b = False: b as (k, n), transposed by the package into its own scratch
    say(f"schema gemm_a8w8 row_major trans_b=False m={m} n={n} k={k}")
    op = _op("gemm_a8w8_blockwise_scaled@1.0", "row_major")
    q, s, b, bs = _fp8_operands(m, n, k, seed=m + 9)
    a_scale = s.t().contiguous()
    out = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    op(a=q, b=b.t().contiguous(), a_scale=a_scale, b_scale=bs, scale_major_mode="K", trans_b=False,
       operand_format="none:none", bias=None, out_dtype=None, out=out)
    ref = aklr_amd.gemm_a8w8_blockwise_scaled(q, b, a_scale, bs)
    torch.cuda.synchronize()
    assert _same(out, ref)


@pytest.mark.parametrize("m,n,k", [(4, 2112, 7168), (200, 1024, 4096)])
def test_gemm_a4w4_b_shuffled_package(m, n, k):
    say(f"schema gemm_a4w4 b_shuffled m={m} n={n} k={k}")
    op = _op("gemm_a4w4_mxfp4@1.0", "b_shuffled")
    x = workloads.activations(m, k, seed=m + 3, device=DEV)
    qa, sa = aklr_amd.dynamic_mxfp4_quant(x, shuffle=True)
    wb, sb = workloads.mxfp4_weight(n, k, seed=m + 4, device=DEV)
    bb, sbb = layouts.shuffle_weight(wb), layouts.e8m0_scales(sb)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    op(a=qa, b=bb, a_scale=sa, b_scale=sbb, trans_b=True, operand_format="none:preshuffled", alpha=1.0, beta=0.0,
       bias=None, out_dtype=None, out=out)
    ref = aklr_amd.gemm_a4w4_mxfp4(qa, bb, sa, sbb)
    torch.cuda.synchronize()
    assert _same(out, ref)


@pytest.mark.parametrize("t", [33, 400])
def test_deepseek_v2_fp8_moe_package(t):
    # the contract's attr values (topk 8 of 8 groups, 4 kept); the op declines others
    e, d, inter, topk, groups, topk_group = 32, 512, 256, 8, 8, 4
    say(f"schema deepseek_v2_fp8_moe shuffled_16x16 t={t} e={e} d={d} inter={inter}")
    op = _op("deepseek_v2_fp8_moe@1.0", "shuffled_16x16")
    g = workloads.generator(t, DEV)
    x = torch.randn((t, d), generator=g, device=DEV).to(torch.bfloat16)
    router = (torch.randn((e, d), generator=g, device=DEV) * 0.05).to(torch.bfloat16)
    bias = (torch.randn((e,), generator=g, device=DEV) * 0.05).to(torch.bfloat16)
    w1 = (torch.randn((e + 1, 2 * inter, d), generator=g, device=DEV) * 64).clamp(-448, 448).to(torch.float8_e4m3fn)
    w2 = (torch.randn((e + 1, d, inter), generator=g, device=DEV) * 64).clamp(-448, 448).to(torch.float8_e4m3fn)
    s1 = torch.exp2(torch.rand((e + 1, 2 * inter // 128, d // 128), generator=g, device=DEV) * -3) / 512
    s2 = torch.exp2(torch.rand((e + 1, d // 128, inter // 128), generator=g, device=DEV) * -3) / 512
    w1s, w2s = layouts.shuffle_weight(w1), layouts.shuffle_weight(w2)
    out = torch.empty((t, d), dtype=torch.bfloat16, device=DEV)
    op(hidden_states=x, router_weight=router, correction_bias=bias, w1=w1s, w1_scale=s1, w2=w2s, w2_scale=s2,
       topk=topk, num_expert_group=groups, topk_group=topk_group, renormalize=True, scoring_func="sigmoid",
       routed_scaling_factor=2.5, out_dtype=None, out=out)
    ref = aklr_amd.deepseek_v2_fp8_moe(x, router, bias, w1s, s1, w2s, s2, topk, groups, topk_group, True, "sigmoid",
                                       2.5)
    torch.cuda.synchronize()
    assert isinstance(ref, torch.Tensor), f"not served: {ref}"
    assert _same(out, ref)
    assert torch.isfinite(out.float()).all() and out.float().abs().sum() > 0

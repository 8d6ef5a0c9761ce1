"""Every output of the prefill-size GEMMs, against a float32 restatement of the op on the GPU.

The prefill parity tests in test_gpu_gemm.py compare a seeded sample of rows x columns, which the host
oracle computes; a fault confined to one output tile could fall between the samples. Here the reference
is the op's definition -- dequantize both operands to float32 (block scales applied), then one float32
matmul -- computed by torch on the GPU with TF32 off. That reference is itself checked against the
oracle on a seeded sample of rows x columns first (to 1e-4 of the output rms: two float32 matmuls that
sum in different orders), so it is pinned to the same semantics
(oracle/gemm.py: gemm_a8w8_blockwise_scaled, gemm_a4w4_mxfp4). Then every element of the product's
output is compared with it:
- FP8: the north-star tolerance |out - y| <= 1e-2 * rms(y) + 1e-2 * |y| and the contract's
  ToleranceBound (atol 1e-2, rtol 1e-2 + bf16 unit roundoff 2**-8), as in test_gpu_gemm.py;
- MXFP4: the contract's DotProductBound(max_split_k=1), with M the same matmul over the operands'
  absolute values, and its bias test |mean(err)| / rms(err) <= 5 / sqrt(size).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import aklr_amd
from aklr_amd import layouts, workloads
from oracle import gemm as ogemm
from tests.helpers import f32, say, u8

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
E2M1 = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)


@pytest.fixture(autouse=True)
def _fp32_matmul():
    prev = torch.get_float32_matmul_precision()
    torch.set_float32_matmul_precision("highest")  # no TF32 / xf32 in the reference
    yield
    torch.set_float32_matmul_precision(prev)


def _sample(m, n, rows=48, cols=384, seed=0):
    rng = np.random.default_rng(seed)
    return np.sort(rng.choice(m, min(m, rows), replace=False)), np.sort(rng.choice(n, min(n, cols), replace=False))


def _fp8_dequant(codes, scales_rows_by_block):
    """codes [r, k] fp8, scales [r, k / 128] float32 -> float32 [r, k]."""
    r, k = codes.shape
    return (codes.float().view(r, k // 128, 128) * scales_rows_by_block.unsqueeze(-1)).view(r, k)


def _fp4_dequant(packed, e8m0):
    """packed e2m1 bytes [r, k / 2] (low nibble first), e8m0 scales [r, k / 32] -> float32 [r, k]."""
    r, k2 = packed.shape
    table = torch.tensor(E2M1, dtype=torch.float32, device=packed.device)
    p = packed.view(torch.uint8).long()
    vals = torch.stack([table[p & 0xF], table[p >> 4]], dim=-1).view(r, 2 * k2)
    scale = torch.ldexp(torch.ones((), device=packed.device), e8m0.view(torch.uint8).float() - 127.0)
    return (vals.view(r, -1, 32) * scale.unsqueeze(-1)).view(r, 2 * k2)


def _assert_all_within(out, ref, what):
    got = out.double()
    y = ref.double()
    err = (got - y).abs()
    rms = float(y.pow(2).mean().sqrt()) or 1.0
    north = err <= 1e-2 * rms + 1e-2 * y.abs()
    contract = err <= 1e-2 + (1e-2 + 2.0**-8) * y.abs()
    bad_n, bad_c = int((~north).sum()), int((~contract).sum())
    say(f"  {what}: max|err|/rms {float(err.max()) / rms:.3e}, outside north star {bad_n}, outside contract {bad_c}")
    assert bad_n == 0, f"{what}: {bad_n} outputs outside the north-star tolerance"
    assert bad_c == 0, f"{what}: {bad_c} outputs outside the contract ToleranceBound"


FP8_CASES = [(1024, "b_shuffled"), (4096, "b_shuffled"), (8192, "row_major")]


@pytest.mark.parametrize("nk", workloads.DEEPSEEK_NK)
@pytest.mark.parametrize("m,variant", FP8_CASES)
def test_fp8_prefill_every_output(m, variant, nk):
    n, k = nk
    say(f"gemm_a8w8 full output m={m} n={n} k={k} {variant}")
    x = workloads.activations(m, k, seed=m + 41, device=DEV)
    q, s = aklr_amd.per_group_quant_fp8(x)  # s: [k / 128, m]
    b, bs = workloads.blockwise_fp8_weight(n, k, seed=m + 42, device=DEV)
    if variant == "b_shuffled":
        out = aklr_amd.gemm_a8w8_blockwise_scaled(q, layouts.shuffle_weight(b), s.view(m, k // 128), bs,
                                                  operand_format="none:preshuffled")
    else:
        out = aklr_amd.gemm_a8w8_blockwise_scaled(q, b, s.t().contiguous(), bs)
    assert isinstance(out, torch.Tensor), f"not served: {out}"
    a32 = _fp8_dequant(q, s.t())
    b32 = _fp8_dequant(b, bs.repeat_interleave(128, dim=0)[:n])
    ref = a32 @ b32.t()
    torch.cuda.synchronize()
    del a32, b32
    # the GPU reference against the oracle on a sample
    r, c = _sample(m, n, seed=m)
    ora = ogemm.gemm_a8w8_blockwise_scaled(u8(q), u8(b), s.cpu().numpy(), bs.cpu().numpy(), scale_major_mode="MN",
                                           rows=r, cols=c)
    ref_s = ref[torch.from_numpy(r).to(DEV)][:, torch.from_numpy(c).to(DEV)].cpu().numpy()
    gap = float(np.abs(ref_s - ora).max() / (np.sqrt(np.mean(ora.astype(np.float64) ** 2)) or 1.0))
    assert gap < 1e-4, f"GPU float32 reference disagrees with the oracle: {gap:.3e} of rms"
    _assert_all_within(out, ref, f"m={m} n={n} k={k} {variant}")


@pytest.mark.parametrize("nk", workloads.LLAMA70B_NK)
@pytest.mark.parametrize("m", [512, 4096])
def test_mxfp4_prefill_every_output(m, nk):
    n, k = nk
    say(f"gemm_a4w4_mxfp4 full output m={m} n={n} k={k}")
    x = workloads.activations(m, k, seed=m + 51, device=DEV)
    qa, sa = aklr_amd.dynamic_mxfp4_quant(x, shuffle=True)
    qa_rm, sa_rm = aklr_amd.dynamic_mxfp4_quant(x, shuffle=False)
    wb, sb = workloads.mxfp4_weight(n, k, seed=m + 52, device=DEV)
    out = aklr_amd.gemm_a4w4_mxfp4(qa, layouts.shuffle_weight(wb), sa, layouts.e8m0_scales(sb))
    assert isinstance(out, torch.Tensor), f"not served: {out}"
    a32 = _fp4_dequant(qa_rm, sa_rm)
    b32 = _fp4_dequant(wb, sb)
    ref = a32 @ b32.t()
    mag = a32.abs() @ b32.abs().t()
    torch.cuda.synchronize()
    del a32, b32
    r, c = _sample(m, n, seed=m + 1)
    ora = ogemm.gemm_a4w4_mxfp4(u8(qa_rm), u8(wb), u8(sa_rm), u8(sb), rows=r, cols=c)
    ri, ci = torch.from_numpy(r).to(DEV), torch.from_numpy(c).to(DEV)
    ref_s = ref[ri][:, ci].cpu().numpy()
    gap = float(np.abs(ref_s - ora).max() / (np.sqrt(np.mean(ora.astype(np.float64) ** 2)) or 1.0))
    assert gap < 1e-4, f"GPU float32 reference disagrees with the oracle: {gap:.3e} of rms"
    # DotProductBound(max_split_k=1), restated on the GPU from oracle/gemm.py: dot_product_bound
    n_eff = k  # max_split_k = 1: ceil(k / 1) + bit_length(0)
    multiple = 6.0 * math.sqrt(n_eff) + 2.0
    y = ref.double()
    err = out.double() - y
    bound = 2.0 * multiple * ogemm.FP32_UNIT_ROUNDOFF * mag.double().abs() + ogemm.OUT_UNIT_ROUNDOFF["bfloat16"] * y.abs()
    bad = int((err.abs() > bound).sum())
    peak = float((err.abs() / bound).max())
    rms = float(err.pow(2).mean().sqrt())
    bias = abs(float(err.mean())) / rms if rms else 0.0
    say(f"  DotProductBound peak multiple {peak:.3f}, outside {bad}, |mean|/rms {bias:.2e}")
    assert bad == 0, f"mxfp4 m={m} n={n} k={k}: {bad} outputs outside DotProductBound"
    assert bias <= 5.0 / math.sqrt(err.numel()), f"mxfp4 m={m} n={n} k={k}: biased errors ({bias:.2e})"
    # the host check on the same sample, through the oracle's own bound function
    got = f32(out)[np.ix_(r, c)]
    mag_s = ogemm.gemm_a4w4_mxfp4(u8(qa_rm) & 0x77, u8(wb) & 0x77, u8(sa_rm), u8(sb), rows=r, cols=c)
    assert ogemm.within_dot_product_bound(got, ora, mag_s, k)

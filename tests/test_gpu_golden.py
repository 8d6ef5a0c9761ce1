"""The HIP kernels on the golden fixtures of tests/golden/ (independent torch restatement and
float64 products): quantizers bit-exact, GEMMs within the north-star tolerance of the float64
product, through the row-major and aiter-preshuffled layouts."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import aklr_amd
from aklr_amd import layouts
from oracle import gemm as ogemm
from oracle import layouts as olay
from tests.helpers import assert_same_bits, f32, say, u8

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("name", sorted(p.name for p in GOLDEN.glob("quant_*.npz")))
def test_quant_golden(name):
    say(f"golden quant {name}")
    g = _load(name)
    x = torch.from_numpy(g["x_bf16_bits"].view(np.int16)).view(torch.bfloat16).to(DEV)
    q, s = aklr_amd.per_group_quant_fp8(x)
    qm, sm = aklr_amd.per_group_quant_mxfp8(x)
    q4, s4 = aklr_amd.dynamic_mxfp4_quant(x)
    q4s, s4s = aklr_amd.dynamic_mxfp4_quant(x, shuffle=True)
    torch.cuda.synchronize()
    assert_same_bits(u8(q), g["fp8_codes"], "fp8 codes")
    assert_same_bits(s.cpu().numpy(), g["fp8_scales"], "fp8 scales")
    assert_same_bits(u8(qm), g["mxfp8_codes"], "mxfp8 codes")
    assert_same_bits(u8(sm), g["mxfp8_scales"], "mxfp8 scales")
    assert_same_bits(u8(q4), g["mxfp4_packed"], "mxfp4 codes")
    assert_same_bits(u8(s4), g["mxfp4_scales"], "mxfp4 scales")
    assert_same_bits(u8(q4s), g["mxfp4_packed"], "mxfp4 codes (shuffled call)")
    assert_same_bits(u8(s4s), olay.e8m0_scales(g["mxfp4_scales"]), "mxfp4 shuffled scales")


def _check(out, want, what):
    got = f32(out)
    assert ogemm.within_north_star(got, want), f"{what}: max|err|/rms {ogemm.rms_normalized_error(got, want)[0]:.3e}"


@pytest.mark.parametrize("name", sorted(p.name for p in GOLDEN.glob("gemm8_*.npz")))
def test_gemm8_golden(name):
    say(f"golden gemm8 {name}")
    g = _load(name)
    a = torch.from_numpy(g["a"]).view(torch.float8_e4m3fn).to(DEV)
    b = torch.from_numpy(g["b"]).view(torch.float8_e4m3fn).to(DEV)
    sgm = torch.from_numpy(g["a_scale_group_major"]).to(DEV)
    sb = torch.from_numpy(g["b_scale"]).to(DEV)
    m, k = a.shape
    out = aklr_amd.gemm_a8w8_blockwise_scaled(a, b, sgm.t().contiguous(), sb)
    out_mn = aklr_amd.gemm_a8w8_blockwise_scaled(a, b, sgm, sb, scale_major_mode="MN")
    out_sh = aklr_amd.gemm_a8w8_blockwise_scaled(a, layouts.shuffle_weight(b), sgm.view(m, k // 128), sb,
                                                 operand_format="none:preshuffled")
    torch.cuda.synchronize()
    for o, what in ((out, "row_major K"), (out_mn, "row_major MN"), (out_sh, "b_shuffled")):
        assert isinstance(o, torch.Tensor), f"{what}: not served ({o})"
        _check(o, g["out_f64"], f"{name} {what}")


@pytest.mark.parametrize("name", sorted(p.name for p in GOLDEN.glob("gemm4_*.npz")))
def test_gemm4_golden(name):
    say(f"golden gemm4 {name}")
    g = _load(name)
    t = {k: torch.from_numpy(g[k]).to(DEV) for k in ("a", "b", "a_scale", "b_scale")}
    out = aklr_amd.gemm_a4w4_mxfp4(t["a"], t["b"], t["a_scale"], t["b_scale"], operand_format="none:none")
    n = t["b"].shape[0]
    if n % 16 == 0 and t["b"].shape[1] % 32 == 0:
        out_sh = aklr_amd.gemm_a4w4_mxfp4(t["a"], layouts.shuffle_weight(t["b"]), layouts.e8m0_scales(t["a_scale"]),
                                          layouts.e8m0_scales(t["b_scale"]))
    else:
        out_sh = None
    torch.cuda.synchronize()
    _check(out, g["out_f64"], f"{name} row_major")
    if out_sh is not None:
        _check(out_sh, g["out_f64"], f"{name} b_shuffled")

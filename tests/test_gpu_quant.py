"""GPU parity of the activation quantizers against the CPU oracle: codes and scales bit-exact.

Covers config 1 (32 x 2048), the decode/prefill activation shapes of configs 2/3 (with 1% x20
outliers), an exhaustive sweep of every bf16 value |v| <= 448 through a unit scale (every e4m3 rounding
case, ties and subnormals included), all-zero and denormal groups, the largest hidden size, and the
MXFP8 / MXFP4 quantizers (row-major and aiter-shuffled scales).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import aklr_amd
from aklr_amd import workloads
from oracle import formats as ofmt
from oracle import layouts as olay
from oracle import quant as oquant
from tests.helpers import assert_same_bits, bf16_bits, say, u8

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _check_fp8(x: torch.Tensor, what: str) -> None:
    say(f"per_group_quant_fp8 {what} shape={tuple(x.shape)}")
    q, s = aklr_amd.per_group_quant_fp8(x)
    torch.cuda.synchronize()
    assert q.dtype == torch.float8_e4m3fn and s.dtype == torch.float32
    assert tuple(s.shape) == (x.shape[1] // 128, x.shape[0])
    q_ref, s_ref = oquant.per_group_quant_fp8(bf16_bits(x))
    assert_same_bits(u8(q), q_ref, f"{what} codes")
    assert_same_bits(s.cpu().numpy(), s_ref, f"{what} scales")


def test_fp8_config1():
    _check_fp8(workloads.activations(32, 2048, seed=0, device=DEV, outliers=False), "config1")


@pytest.mark.parametrize("k", [7168, 1536, 16384])
@pytest.mark.parametrize("m", [1, 4, 16, 64, 128, 1024])
def test_fp8_deepseek_shapes(m, k):
    _check_fp8(workloads.activations(m, k, seed=m + k, device=DEV), f"deepseek m={m} k={k}")


def test_fp8_large_prefill():
    _check_fp8(workloads.activations(8192, 7168, seed=5, device=DEV), "prefill 8192x7168")


def test_fp8_every_bf16_value_through_unit_scale():
    # amax 448 gives s = 448 * fl32(1/448) == 1.0 exactly, so each value is rounded to e4m3 as it is.
    assert np.float32(448.0) * oquant.INV448 == np.float32(1.0)
    bits = np.arange(0, 0x8000, dtype=np.uint16)
    vals = ofmt.bf16_bits_to_f32(bits)
    keep = bits[np.isfinite(vals) & (np.abs(vals) <= 448.0)]
    allbits = np.concatenate([keep, keep | 0x8000])
    per_row = 127
    rows = -(-allbits.size // per_row)
    data = np.zeros((rows, 128), dtype=np.uint16)
    data[:, 0] = 0x43E0  # 448.0
    flat = np.zeros(rows * per_row, dtype=np.uint16)
    flat[: allbits.size] = allbits
    data[:, 1:] = flat.reshape(rows, per_row)
    x = torch.from_numpy(data.view(np.int16)).view(torch.bfloat16).to(DEV)
    _check_fp8(x, "every bf16 value")


def test_fp8_edge_groups():
    # zero group, denormal-only group, a single huge value, max hidden size, one row
    x = workloads.activations(3, 21504, seed=9, device=DEV)
    x[0, :128] = 0
    x[1, 128:256] = torch.tensor(1e-39, dtype=torch.float32).to(torch.bfloat16)
    x[2, 256] = 3.0e38
    _check_fp8(x, "edge groups")
    _check_fp8(workloads.activations(1, 128, seed=2, device=DEV), "1x128")


def test_fp8_deterministic():
    x = workloads.activations(256, 7168, seed=4, device=DEV)
    q1, s1 = aklr_amd.per_group_quant_fp8(x)
    q2, s2 = aklr_amd.per_group_quant_fp8(x)
    assert torch.equal(q1.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(s1, s2)


@pytest.mark.parametrize("m,k", [(3, 256), (32, 2048), (128, 7168), (4096, 7168)])
def test_mxfp8(m, k):
    x = workloads.activations(m, k, seed=m, device=DEV)
    say(f"per_group_quant_mxfp8 m={m} k={k}")
    q, s = aklr_amd.per_group_quant_mxfp8(x)
    torch.cuda.synchronize()
    q_ref, s_ref = oquant.per_group_quant_mxfp8(bf16_bits(x))
    assert_same_bits(u8(q), q_ref, "mxfp8 codes")
    assert_same_bits(u8(s), s_ref, "mxfp8 scales")


@pytest.mark.parametrize("shuffle", [False, True])
@pytest.mark.parametrize("m,k", [(1, 64), (3, 96), (32, 8192), (300, 1024), (512, 28672)])
def test_mxfp4(m, k, shuffle):
    x = workloads.activations(m, k, seed=m + 1, device=DEV)
    say(f"dynamic_mxfp4_quant m={m} k={k} shuffle={shuffle}")
    q, s = aklr_amd.dynamic_mxfp4_quant(x, shuffle=shuffle)
    torch.cuda.synchronize()
    q_ref, s_ref = oquant.dynamic_mxfp4_quant(bf16_bits(x))
    assert_same_bits(u8(q), q_ref, "mxfp4 codes")
    if shuffle:
        s_ref = olay.e8m0_scales(s_ref, shuffled=True)
    assert_same_bits(u8(s), s_ref, "mxfp4 scales")


def test_mxfp4_every_bf16_value_through_unit_scale():
    # A 32-value block whose amax is 6.0 gets E = 0 (frexp(6) = (0.75, 3): 3 - 3 + (0.75 > 0.75) = 0), a
    # unit scale, so each value is rounded to e2m1 as it is: every finite bf16 value of magnitude <= 6
    # (both signs, zeros and subnormals included) goes through the kernel's conversion once and must
    # give the oracle's nibble (midpoints to the even code, sign kept).
    bits = np.arange(0, 0x40C1, dtype=np.uint16)  # +0 .. 6.0
    assert ofmt.bf16_bits_to_f32(np.array([0x40C0], np.uint16))[0] == 6.0
    allbits = np.concatenate([bits, bits | 0x8000])
    per_block = 31
    blocks = -(-allbits.size // per_block)
    rows = -(-blocks // 32)  # 32 blocks per row of 1024 values
    data = np.zeros((rows * 32, 32), dtype=np.uint16)
    data[:, 0] = 0x40C0  # 6.0 in every block
    flat = np.zeros(rows * 32 * per_block, dtype=np.uint16)
    flat[: allbits.size] = allbits
    data[:, 1:] = flat.reshape(rows * 32, per_block)
    x = torch.from_numpy(data.reshape(rows, 1024).view(np.int16)).view(torch.bfloat16).to(DEV)
    say(f"dynamic_mxfp4_quant every bf16 |v| <= 6: {allbits.size} values in {rows} rows")
    q, s = aklr_amd.dynamic_mxfp4_quant(x)
    torch.cuda.synchronize()
    q_ref, s_ref = oquant.dynamic_mxfp4_quant(data.reshape(rows, 1024))
    assert np.all(s_ref == 127)
    assert_same_bits(u8(s), s_ref, "mxfp4 unit scales")
    assert_same_bits(u8(q), q_ref, "mxfp4 codes of every bf16 value")


def test_mxfp4_matches_weight_quantizer():
    # the torch weight quantizer of aklr_amd.workloads and the GPU activation kernel implement the same rule
    x = workloads.activations(64, 4096, seed=11, device=DEV)
    q, s = aklr_amd.dynamic_mxfp4_quant(x)
    q2, s2 = workloads.mxfp4_quantize(x)
    assert torch.equal(q.view(torch.uint8), q2) and torch.equal(s.view(torch.uint8), s2)

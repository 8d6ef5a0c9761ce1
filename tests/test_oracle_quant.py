"""Pins oracle/quant.py with checks a plausible mistake would fail:

- per_group_quant_fp8: the constant fl32(1/448) bit pattern; the scale as the correctly rounded
  product amax * fl32(1/448) (exact float64 product, then one rounding) -- which differs from
  amax / 448 on inputs found here, so a divide fails; inv the correctly rounded reciprocal; codes
  as torch's e4m3fn cast of the exactly computed x * inv; the group's amax element landing on
  exactly +-448; the all-zero group; sign symmetry; the half-ulp dequant bound; group-major scales.
- per_group_quant_mxfp8: the scale as the least power of two >= fl32(amax * fl32(1/448)) (exact
  frexp arithmetic); codes as torch's cast of x / 2**E.
- dynamic_mxfp4_quant: E as the least integer with amax / 2**E <= 6 (brute-force search over E, the
  closed form of frexp(amax) -> e - 3 + (m > 0.75)); codes by brute-force nearest search; NaN blocks.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import formats as f
from oracle import quant as q


def _bf16(x) -> np.ndarray:
    return f.f32_to_bf16_bits(np.asarray(x, dtype=np.float32))


def _rows(seed, rows, cols, outliers=True):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    if outliers:
        x = np.where(rng.random((rows, cols)) < 0.01, x * 20, x)
    return _bf16(x)


def test_inv448_constant():
    # 1/448 = 2**-9 * 1.142857...; 1.142857 * 2**23 = 0x924924.92 -> rounds up to 0x924925
    assert int(q.INV448.view(np.uint32)) == 0x3B124925


def _correct_product(a: np.ndarray, b) -> np.ndarray:
    return (a.astype(np.float64) * np.float64(b)).astype(np.float32)  # exact in f64, one rounding


def test_fp8_scales_are_rounded_products_not_quotients():
    xb = _rows(0, 64, 7168)
    _, s = q.per_group_quant_fp8(xb)
    x = f.bf16_bits_to_f32(xb).reshape(64, 56, 128)
    amax = np.maximum(np.abs(x).max(-1), np.float32(1e-10))
    want = _correct_product(amax, q.INV448).T
    assert np.array_equal(s.view(np.uint32), want.view(np.uint32))
    # the divide differs for some amax here: a quantizer computing amax / 448 would fail the line above
    quotient = (amax.astype(np.float64) / 448.0).astype(np.float32).T
    assert np.any(quotient.view(np.uint32) != want.view(np.uint32))


def test_fp8_codes_from_exact_arithmetic_and_torch_cast():
    xb = _rows(1, 32, 2048)
    codes, s = q.per_group_quant_fp8(xb)
    x = f.bf16_bits_to_f32(xb).reshape(32, 16, 128)
    inv = (1.0 / s.T.astype(np.float64)).astype(np.float32)  # correctly rounded reciprocal
    v = (x.astype(np.float64) * inv[..., None].astype(np.float64)).astype(np.float32)
    v = np.clip(v, -448, 448).astype(np.float32)
    want = torch.from_numpy(v.reshape(32, 2048)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(codes, want)


def test_fp8_amax_element_is_exactly_448_and_group_major():
    rows, cols = 5, 384
    x = np.zeros((rows, cols), dtype=np.float32)
    rng = np.random.default_rng(2)
    expect_amax = np.zeros((cols // 128, rows), dtype=np.float32)
    for r in range(rows):
        for g in range(cols // 128):
            amax = np.float32(2.0 ** (r - g)) * np.float32(1.0 + 0.01 * (r * 3 + g))
            vals = rng.uniform(-1, 1, 128).astype(np.float32) * amax * np.float32(0.9)
            pos = (r * 7 + g * 13) % 128
            vals[pos] = -amax if (r + g) % 2 else amax
            x[r, g * 128:(g + 1) * 128] = vals
    xb = _bf16(x)
    xr = f.bf16_bits_to_f32(xb)
    codes, s = q.per_group_quant_fp8(xb)
    assert s.shape == (cols // 128, rows)  # group-major [H/128, T]; T != H/128 here
    for r in range(rows):
        for g in range(cols // 128):
            grp = xr[r, g * 128:(g + 1) * 128]
            i = int(np.argmax(np.abs(grp)))
            assert codes[r, g * 128 + i] == (0xFE if grp[i] < 0 else 0x7E)
            assert s[g, r] == _correct_product(np.array([abs(grp[i])]), q.INV448)[0]


def test_fp8_zero_group_sign_symmetry_and_bound():
    xb = _rows(3, 8, 1024)
    xb[0, :128] = 0
    codes, s = q.per_group_quant_fp8(xb)
    assert np.all(codes[0, :128] == 0)
    assert s[0, 0] == _correct_product(np.array([1e-10], dtype=np.float32), q.INV448)[0]
    neg = xb ^ np.uint16(0x8000)
    codes_n, s_n = q.per_group_quant_fp8(neg)
    assert np.array_equal(s_n, s)
    nz = codes[1:] != 0
    assert np.array_equal(codes_n[1:][nz], codes[1:][nz] ^ 0x80)
    # |fp8(q) * s - x| <= half an e4m3 ulp of x/s, times s (plus the rounding of x*inv)
    x = f.bf16_bits_to_f32(xb)
    dq = f.fp8_to_f32(codes) * np.repeat(s.T, 128, axis=1)
    v = np.abs(x) / np.repeat(s.T, 128, axis=1)
    ulp = np.where(v < 2.0**-6, 2.0**-9, np.exp2(np.floor(np.log2(np.maximum(v, 2.0**-6))) - 3))
    bound = (0.5 * ulp + 4 * v * 2.0**-24) * np.repeat(s.T, 128, axis=1)
    assert np.all(np.abs(dq - x) <= bound)


def test_mxfp8_scale_is_least_power_of_two():
    xb = _rows(4, 16, 2048)
    xb[0, :32] = 0
    codes, e = q.per_group_quant_mxfp8(xb)
    x = f.bf16_bits_to_f32(xb).reshape(16, 64, 32)
    amax = np.maximum(np.abs(x).max(-1), np.float32(1e-10))
    target = _correct_product(amax, q.INV448)
    for (r, g), t in np.ndenumerate(target):
        mant, ex = math.frexp(float(t))  # t = mant * 2**ex, mant in [0.5, 1)
        least = ex - 1 if mant == 0.5 else ex  # least k with 2**k >= t
        assert int(e[r, g]) - 127 == least
    scale = np.exp2(e.astype(np.float64) - 127)
    v = np.clip(x.astype(np.float64) / scale[..., None], -448, 448).astype(np.float32)
    want = torch.from_numpy(v.reshape(16, 2048)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(codes, want)


def _least_exponent(amax: float) -> int:
    e = -200
    while amax / 2.0**e > 6.0:
        e += 1
    while e > -200 and amax / 2.0 ** (e - 1) <= 6.0:
        e -= 1
    return max(-127, min(127, e))


@pytest.mark.parametrize("seed", [5, 6])
def test_mxfp4_exponent_and_codes_bruteforce(seed):
    xb = _rows(seed, 6, 512)
    xb[0, :32] = 0  # all-zero block: amax floored at 1e-10
    x = f.bf16_bits_to_f32(xb)
    x[1, 32:64] = np.float32(6.0) * np.float32(2.0**-3)  # amax exactly 6 * 2**k: the boundary of the rule
    x[1, 64:96] = np.float32(6.0000005)
    xb = _bf16(x)
    x = f.bf16_bits_to_f32(xb)
    packed, sb = q.dynamic_mxfp4_quant(xb)
    nib = f.unpack_nibbles(packed)
    for r in range(x.shape[0]):
        for g in range(x.shape[1] // 32):
            blk = x[r, g * 32:(g + 1) * 32]
            amax = max(float(np.abs(blk).max()), float(np.float32(1e-10)))
            E = _least_exponent(amax)
            assert int(sb[r, g]) == E + 127, (r, g, amax)
            for i, v in enumerate(blk):
                sv = float(v) / 2.0**E
                best, bestd = 0, float("inf")
                for c, gval in enumerate(f.E2M1_GRID):
                    d = abs(abs(sv) - float(gval))
                    if d < bestd or (d == bestd and c % 2 == 0):
                        best, bestd = c, d
                want = best | (8 if np.signbit(v) else 0)
                assert nib[r, g * 32 + i] == want, (r, g, i, v)
    assert sb[1, 1] == 127 - 3  # amax 0.75 = 6 * 2**-3: E = -3 (0.75 / 2**-3 = 6 <= 6)


def test_mxfp4_non_finite_block():
    x = np.ones((1, 64), dtype=np.float32)
    x[0, 3] = np.inf
    packed, sb = q.dynamic_mxfp4_quant(_bf16(x))
    assert sb[0, 0] == 255 and np.all(packed[0, :16] == 0)
    assert sb[0, 1] == 127 - 2  # amax 1: frexp -> (0.5, 1): E = 1 - 3 = -2

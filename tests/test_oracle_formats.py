"""Pins oracle/formats.py: element decodings against torch's own dtypes (library casts), e4m3fn
rounding against torch's cast over every bf16 value and 2**20 random fp32 values, e2m1 rounding
against a brute-force nearest search, and hand-worked codes."""
from __future__ import annotations

import numpy as np
import torch

from oracle import formats as f


def _torch_decode(dtype):
    return torch.arange(256, dtype=torch.uint8).view(dtype).float().numpy()


def test_e4m3fn_table_matches_torch():
    want = _torch_decode(torch.float8_e4m3fn)
    assert np.array_equal(np.isnan(f.E4M3FN_TABLE), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(f.E4M3FN_TABLE[ok].view(np.uint32), want[ok].view(np.uint32))
    # hand-worked: 0x7E = 448, 0x01 = 2**-9 (smallest subnormal), 0x08 = 2**-6, 0x38 = 1
    assert f.E4M3FN_TABLE[0x7E] == 448 and f.E4M3FN_TABLE[0x01] == 2.0**-9
    assert f.E4M3FN_TABLE[0x08] == 2.0**-6 and f.E4M3FN_TABLE[0x38] == 1.0 and f.E4M3FN_TABLE[0xB8] == -1.0


def test_e5m2_table_matches_torch():
    want = _torch_decode(torch.float8_e5m2)
    assert np.array_equal(np.isnan(f.E5M2_TABLE), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(f.E5M2_TABLE[ok], want[ok])


def _torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).view(
        torch.uint8).numpy()


def test_e4m3fn_rounding_every_bf16_value():
    bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    x = f.bf16_bits_to_f32(bits)
    x = x[np.isfinite(x)]
    assert np.array_equal(f.f32_to_e4m3fn(x), _torch_e4m3(x))


def test_e4m3fn_rounding_random_fp32():
    rng = np.random.default_rng(0)
    # magnitudes 2**-14 .. 2**10 (subnormal range, ties, overflow to NaN) and arbitrary low bits
    u = rng.integers(0, 1 << 31, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    u = (u & np.uint32(0x807FFFFF)) | (rng.integers(113, 138, size=u.size).astype(np.uint32) << 23)
    x = u.view(np.float32)
    assert np.array_equal(f.f32_to_e4m3fn(x), _torch_e4m3(x))
    # exact ties between neighbouring codes go to the even code
    ties = np.array([1.0 + 1 / 16, 1.0 + 3 / 16, 2.0**-9 * 0.5, 2.0**-9 * 1.5, 464.0, -464.0], dtype=np.float32)
    assert list(f.f32_to_e4m3fn(ties)) == [0x38, 0x3A, 0x00, 0x02, 0x7E, 0xFE]


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(1 << 16) * np.exp2(rng.integers(-40, 40, 1 << 16))).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(f.f32_to_bf16_bits(x), want)


def _nearest_bruteforce(v: float) -> int:
    m = abs(v)
    best, bestd = -1, float("inf")
    for i, g in enumerate(f.E2M1_GRID):
        d = abs(m - float(g))
        if d < bestd or (d == bestd and i % 2 == 0):
            best, bestd = i, d
    return best | (8 if np.signbit(np.float32(v)) else 0)


def test_e2m1_rounding_bruteforce():
    vals = np.concatenate([np.arange(-7.0, 7.0, 1 / 64), f.E2M1_GRID[1:] - 0.0, (f.E2M1_GRID[1:] + f.E2M1_GRID[:-1]) / 2,
                           -(f.E2M1_GRID[1:] + f.E2M1_GRID[:-1]) / 2]).astype(np.float32)
    got = f.e2m1_nibble(vals)
    want = np.array([_nearest_bruteforce(float(v)) for v in vals], dtype=np.uint8)
    assert np.array_equal(got, want)


def test_e2m1_hand_worked_ties():
    # midpoints 0.25 .75 1.25 1.75 2.5 3.5 5 round to the even code: 0, 1.0, 1.0, 2.0, 2.0, 4.0, 4.0
    mids = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 7.0], dtype=np.float32)
    assert list(f.e2m1_nibble(mids)) == [0, 2, 2, 4, 4, 6, 6, 7]
    assert list(f.e2m1_nibble(-mids)) == [8, 10, 10, 12, 12, 14, 14, 15]


def test_e2m1_packing_low_nibble_first():
    # 0x21: low nibble 1 (0.5) first, then 2 (1.0); 0x9F: low F (-6), high 9 (-0.5)
    assert list(f.fp4x2_to_f32(np.array([0x21, 0x9F], dtype=np.uint8))) == [0.5, 1.0, -6.0, -0.5]
    nib = np.array([[1, 2, 15, 9]], dtype=np.uint8)
    assert list(f.pack_nibbles(nib)[0]) == [0x21, 0x9F]
    assert np.array_equal(f.unpack_nibbles(f.pack_nibbles(nib)), nib)


def test_e8m0_matches_torch():
    want = _torch_decode(torch.float8_e8m0fnu)
    got = f.e8m0_to_f32(np.arange(256, dtype=np.uint8))
    assert np.array_equal(np.isnan(got), np.isnan(want)) and np.isnan(got[255])
    assert np.array_equal(got[:255], want[:255])
    assert got[127] == 1.0 and got[0] == 2.0**-127 and got[254] == 2.0**127

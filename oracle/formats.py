"""Element formats of the path, in numpy (test infrastructure; see ``oracle/__init__.py``).

Decoding follows aklr/core/contract/semantics/_dtypes.py:55-110:
- e4m3fn / e5m2: IEEE-style minifloats (``cast`` decoding); e4m3fn has no infinity, 0x7F/0xFF NaN;
- e2m1: nibble table (0, .5, 1, 1.5, 2, 3, 4, 6, then the negatives), two codes per byte, LOW NIBBLE
  FIRST (_dtypes.py:96-100);
- e8m0: 2**(byte - 127), byte 255 NaN (_dtypes.py:60, :101-108).

Encoding fp32 -> e4m3fn is round-to-nearest-even with subnormals, as torch's ``.to(float8_e4m3fn)``
which the reference calls (aklr/ops/quant/reference.py:27). Pinned in tests/test_oracle_formats.py
against torch's cast over every bf16 value and 2**20 random fp32 values, and by hand-worked codes.

Encoding to e2m1 is nearest grid point, ties to the even code (aklr/ops/fused_moe/reference.py:31-36).
Pinned against a brute-force nearest search over the grid and hand-worked ties.
"""
from __future__ import annotations

import numpy as np

E2M1_GRID = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)


# ---------------------------------------------------------------------------------------------
# bf16
def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 (exact)."""
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# ---------------------------------------------------------------------------------------------
# fp8 decode tables
def _e4m3fn_table() -> np.ndarray:
    t = np.empty(256, dtype=np.float32)
    for c in range(256):
        s, e, m = c >> 7, (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            v = np.nan
        elif e == 0:
            v = m * 2.0**-9
        else:
            v = (1.0 + m / 8.0) * 2.0 ** (e - 7)
        t[c] = -v if s else v
    return t


def _e5m2_table() -> np.ndarray:
    t = np.empty(256, dtype=np.float32)
    for c in range(256):
        s, e, m = c >> 7, (c >> 2) & 31, c & 3
        if e == 31:
            v = np.inf if m == 0 else np.nan
        elif e == 0:
            v = m * 2.0**-16
        else:
            v = (1.0 + m / 4.0) * 2.0 ** (e - 15)
        t[c] = -v if s else v
    return t


E4M3FN_TABLE = _e4m3fn_table()
E5M2_TABLE = _e5m2_table()


def fp8_to_f32(codes: np.ndarray, fmt: str = "e4m3fn") -> np.ndarray:
    table = {"e4m3fn": E4M3FN_TABLE, "e5m2": E5M2_TABLE}[fmt]
    return table[np.asarray(codes, dtype=np.uint8)]


def f32_to_e4m3fn(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn codes (uint8), round to nearest even, subnormals kept; |x| rounding past
    448 gives NaN (0x7F/0xFF) as torch's cast does.

    Normal range (|x| >= 2**-6): keep 3 of the 23 fraction bits of the fp32 pattern, rounding to
    nearest even on the integer pattern (a carry moves into the exponent), then rebias 127 -> 7.
    Subnormal range: the multiple of 2**-9 nearest |x|, ties to even (np.rint)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    sign = (u >> 31).astype(np.uint8) << 7
    a = u & np.uint32(0x7FFFFFFF)
    lsb = (a >> 20) & 1
    rounded = (a.astype(np.int64) + 0x7FFFF + lsb) >> 20  # (exponent << 3) | 3 fraction bits
    normal = rounded - (120 << 3)
    sub = np.rint(np.minimum(np.abs(x), np.float32(1.0)) * np.float32(512.0)).astype(np.int64)  # used below 2**-6 only
    code = np.where(a < np.uint32(0x3C800000), sub, normal)  # 0x3C800000 = 2**-6
    code = np.where((code > 0x7E) | (a > np.uint32(0x7F800000)), 0x7F, code)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


# ---------------------------------------------------------------------------------------------
# e2m1 / e8m0
def e2m1_nibble(x: np.ndarray) -> np.ndarray:
    """float32 values already divided by their block scale (|x| <= 6 expected) -> e2m1 nibbles:
    nearest grid point, ties to the even code; the sign bit is the input's sign bit."""
    x = np.asarray(x, dtype=np.float32)
    m = np.abs(x)
    grid = E2M1_GRID
    lo = np.searchsorted(grid, m, side="right") - 1  # largest code <= m
    lo = np.clip(lo, 0, 7)
    hi = np.minimum(lo + 1, 7)
    below = m - grid[lo]
    above = grid[hi] - m
    up = (above < below) | ((above == below) & (hi % 2 == 0))
    idx = np.where(up, hi, lo).astype(np.uint8)
    sign = (x.view(np.uint32) >> 31).astype(np.uint8)
    return idx | (sign << 3)


def e2m1_decode_nibbles(nib: np.ndarray) -> np.ndarray:
    nib = np.asarray(nib, dtype=np.uint8)
    v = E2M1_GRID[nib & 7]
    return np.where(nib & 8, -v, v).astype(np.float32)


def pack_nibbles(nib: np.ndarray) -> np.ndarray:
    """[..., 2j] in the low nibble, [..., 2j+1] in the high nibble."""
    nib = np.asarray(nib, dtype=np.uint8)
    return (nib[..., 0::2] | (nib[..., 1::2] << 4)).astype(np.uint8)


def unpack_nibbles(packed: np.ndarray) -> np.ndarray:
    packed = np.asarray(packed, dtype=np.uint8)
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = packed & 0xF
    out[..., 1::2] = packed >> 4
    return out


def fp4x2_to_f32(packed: np.ndarray) -> np.ndarray:
    """Packed e2m1 bytes [..., k/2] -> float32 [..., k], low nibble first."""
    return e2m1_decode_nibbles(unpack_nibbles(packed))


def e8m0_to_f32(codes: np.ndarray) -> np.ndarray:
    codes = np.asarray(codes, dtype=np.uint8)
    v = np.ldexp(np.float32(1.0), np.minimum(codes, 254).astype(np.int32) - 127).astype(np.float32)
    return np.where(codes == 255, np.float32(np.nan), v).astype(np.float32)

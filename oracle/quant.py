"""Activation quantizers, restated in numpy float32 (test infrastructure; see ``oracle/__init__.py``).

per_group_quant_fp8 -- aklr/ops/quant/reference.py:9-28. Every step rounds to float32 in this order:
    amax = max|x| over 128 values, floored at fl32(1e-10)          (:21)
    s    = amax * fl32(1/448)        -- a multiply, NOT amax / 448  (:22)
    inv  = 1 / s, correctly rounded (torch's ``1.0 / t`` is reciprocal(t) * 1.0)  (:23)
    q    = e4m3fn_rne(clamp(x * inv, -448, 448))                    (:24-27)
  scales are returned group-major [H/128, T] (:28).
  Pinned by: exact rational recomputation of s and inv (tests/test_oracle_quant.py), the amax element
  landing on exactly +-448, the all-zero group, sign symmetry, and the half-ulp dequant bound.

per_group_quant_mxfp8 -- aklr/ops/quant/reference.py:31-48:
    raw = bits(amax * fl32(1/448)); E = (raw >> 23) + (mantissa != 0); scale = 2**(E - 127)
    q = e4m3fn_rne(clamp(x / scale, -448, 448)); scale byte = E.
  Pinned by: exact rational check that 2**(E-127) is the least power of two >= amax*fl32(1/448).

dynamic_mxfp4_quant -- aklr/ops/fused_moe/reference.py:21-37 (aiter dynamic_mxfp4_quant semantics):
    (m, e) = frexp(amax floored at 1e-10); E = clamp(e - 3 + (m > 0.75), -127, 127); s = 2**E
    code = nearest e2m1 grid point to |x/s|, ties to the even code, with x's sign; byte = E + 127.
  A non-finite amax gives scale NaN (byte 255) and zero codes (:26-30).
  Pinned by: brute-force nearest-grid search, hand-worked blocks, |x/s| <= 6 for every block.
"""
from __future__ import annotations

import numpy as np

from .formats import bf16_bits_to_f32, e2m1_nibble, f32_to_e4m3fn, pack_nibbles

INV448 = np.float32(1.0 / 448.0)
AMAX_FLOOR = np.float32(1e-10)


def _as_f32(x: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) or float32 values -> float32."""
    x = np.asarray(x)
    if x.dtype == np.uint16:
        return bf16_bits_to_f32(x)
    return x.astype(np.float32)


def per_group_quant_fp8(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """x: bf16 bits uint16 [T, H] (or float32 holding bf16 values) ->
    (e4m3fn codes uint8 [T, H], fp32 dequant scales [H/128, T] group-major)."""
    x32 = _as_f32(x)
    rows, cols = x32.shape
    assert cols % 128 == 0
    g = x32.reshape(rows, cols // 128, 128)
    amax = np.maximum(np.abs(g).max(axis=-1), AMAX_FLOOR).astype(np.float32)
    scales = (amax * INV448).astype(np.float32)
    inv = (np.float32(1.0) / scales).astype(np.float32)
    v = (g * inv[..., None]).astype(np.float32)
    v = np.clip(v, np.float32(-448.0), np.float32(448.0))
    q = f32_to_e4m3fn(v).reshape(rows, cols)
    return q, np.ascontiguousarray(scales.T)


def per_group_quant_mxfp8(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """x: bf16 bits [T, H] -> (e4m3fn codes [T, H], e8m0 scale bytes uint8 [T, H/32] row-major)."""
    x32 = _as_f32(x)
    rows, cols = x32.shape
    assert cols % 32 == 0
    g = x32.reshape(rows, cols // 32, 32)
    amax = np.maximum(np.abs(g).max(axis=-1), AMAX_FLOOR).astype(np.float32)
    raw = (amax * INV448).astype(np.float32).view(np.int32)
    expo = (raw >> 23) + ((raw & 0x7FFFFF) != 0).astype(np.int32)
    scale = (expo.astype(np.int32) << 23).view(np.float32)
    v = (g / scale[..., None]).astype(np.float32)
    v = np.clip(v, np.float32(-448.0), np.float32(448.0))
    q = f32_to_e4m3fn(v).reshape(rows, cols)
    return q, expo.astype(np.uint8)


def mxfp4_block_exponent(amax: np.ndarray) -> np.ndarray:
    """E per block (int32, already clamped to [-127, 127]); amax float32, finite."""
    m, e = np.frexp(np.maximum(amax, AMAX_FLOOR).astype(np.float32))
    return np.clip(e - 3 + (m > 0.75).astype(np.int32), -127, 127).astype(np.int32)


def dynamic_mxfp4_quant(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """x: bf16 bits [T, H] -> (packed e2m1 uint8 [T, H/2], e8m0 scale bytes [T, H/32] row-major)."""
    x32 = _as_f32(x)
    rows, cols = x32.shape
    assert cols % 32 == 0
    g = x32.reshape(rows, cols // 32, 32)
    amax = np.abs(g).max(axis=-1)
    finite = np.isfinite(amax)
    expo = mxfp4_block_exponent(np.where(finite, amax, np.float32(0.0)))
    scale = np.ldexp(np.float32(1.0), expo).astype(np.float32)
    scaled = (np.where(finite[..., None], g, np.float32(0.0)) / scale[..., None]).astype(np.float32)
    nib = e2m1_nibble(scaled)
    nib = np.where(finite[..., None], nib, np.uint8(0)).astype(np.uint8)
    packed = pack_nibbles(nib.reshape(rows, cols))
    sbytes = np.where(finite, expo + 127, 255).astype(np.uint8)
    return packed, sbytes

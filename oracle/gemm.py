"""Block-scaled GEMMs, restated in numpy float32 (test infrastructure; see ``oracle/__init__.py``).

gemm_a8w8_blockwise_scaled -- aklr/ops/gemm/reference.py:90-105:
    A = fp8(a) * repeat(a_scale, 128 along k)            (a_scale.mT first when scale_major_mode == MN)
    B = fp8(b) * repeat(b_scale, 128 along n and k)      (tails partial: [:n, :k])
    out = A @ B^T (+ bias), float32
gemm_a4w4_mxfp4 -- aklr/ops/gemm/reference.py:108-122:
    out = alpha * (e2m1(a) * 2**(a_scale-127)) @ (e2m1(b) * 2**(b_scale-127))^T (+ bias)

Both take the operands in their row-major (logical) layout; ``rows``/``cols`` restrict the output to a
sample of rows and columns (the same formula on the sampled operands), so full-size GPU results can be
checked on a subset in seconds.

Pinned (tests/test_oracle_gemm.py): a brute-force float64 triple loop on tiny shapes; all-ones scales
reduce to the plain product of the decoded codes; K = 128 is one block; the partial last b_scale row
(N % 128 != 0); MN-major a_scale equals the K-major one transposed; e2m1 low-nibble-first decoding by
hand-worked bytes.
"""
from __future__ import annotations

import math

import numpy as np

from .formats import e8m0_to_f32, fp4x2_to_f32, fp8_to_f32


def _sel(n: int, idx) -> np.ndarray:
    return np.arange(n) if idx is None else np.asarray(idx)


def dequant_a8(a_codes, a_scale, *, fmt="e4m3fn", scale_major_mode="K", rows=None) -> np.ndarray:
    m, k = a_codes.shape
    r = _sel(m, rows)
    sa = np.asarray(a_scale, dtype=np.float32)
    if scale_major_mode == "MN":
        sa = sa.T
    a = fp8_to_f32(a_codes[r], fmt)
    return (a * np.repeat(sa[r], 128, axis=1)[:, :k]).astype(np.float32)


def dequant_b8(b_codes, b_scale, *, fmt="e4m3fn", cols=None) -> np.ndarray:
    n, k = b_codes.shape
    c = _sel(n, cols)
    sb = np.asarray(b_scale, dtype=np.float32)
    b = fp8_to_f32(b_codes[c], fmt)
    return (b * np.repeat(sb[c // 128], 128, axis=1)[:, :k]).astype(np.float32)


def gemm_a8w8_blockwise_scaled(a_codes, b_codes, a_scale, b_scale, *, fmt="e4m3fn", scale_major_mode="K",
                               bias=None, rows=None, cols=None) -> np.ndarray:
    """a_codes uint8 [M, K], b_codes uint8 [N, K] (trans_b), a_scale fp32 [M, K/128] (K) or
    [K/128, M] (MN), b_scale fp32 [ceil(N/128), K/128], bias fp32 [N] -> fp32 [len(rows), len(cols)]."""
    a = dequant_a8(a_codes, a_scale, fmt=fmt, scale_major_mode=scale_major_mode, rows=rows)
    b = dequant_b8(b_codes, b_scale, fmt=fmt, cols=cols)
    out = np.matmul(a, b.T).astype(np.float32)
    if bias is not None:
        out = out + np.asarray(bias, dtype=np.float32)[_sel(b_codes.shape[0], cols)]
    return out.astype(np.float32)


def dequant_fp4(packed, scales, rows=None) -> np.ndarray:
    r = _sel(packed.shape[0], rows)
    v = fp4x2_to_f32(packed[r])
    s = e8m0_to_f32(np.asarray(scales)[r])
    return (v * np.repeat(s, 32, axis=1)).astype(np.float32)


def gemm_a4w4_mxfp4(a_packed, b_packed, a_scale, b_scale, *, alpha=1.0, bias=None, rows=None,
                    cols=None) -> np.ndarray:
    """a_packed uint8 [M, K/2], b_packed [N, K/2], a_scale/b_scale e8m0 bytes [*, K/32] row-major."""
    a = dequant_fp4(a_packed, a_scale, rows)
    b = dequant_fp4(b_packed, b_scale, cols)
    out = (np.float32(alpha) * np.matmul(a, b.T)).astype(np.float32)
    if bias is not None:
        out = out + np.asarray(bias, dtype=np.float32)[_sel(b_packed.shape[0], cols)]
    return out.astype(np.float32)


def rms_normalized_error(actual: np.ndarray, expected: np.ndarray) -> tuple[float, float]:
    """(max |actual - expected| / rms(expected), rms(expected))."""
    expected = np.asarray(expected, dtype=np.float64)
    rms = float(np.sqrt(np.mean(expected**2))) or 1.0
    err = np.abs(np.asarray(actual, dtype=np.float64) - expected)
    return float(err.max() / rms) if err.size else 0.0, rms


def within_north_star(actual, expected, rtol=1e-2, atol=1e-2) -> bool:
    """|actual - y| <= atol * rms(y) + rtol * |y| elementwise
    (rtol 1e-2 / atol 1e-2 after normalising by the output RMS)."""
    expected = np.asarray(expected, dtype=np.float64)
    rms = float(np.sqrt(np.mean(expected**2))) or 1.0
    err = np.abs(np.asarray(actual, dtype=np.float64) - expected)
    return bool(np.all(err <= atol * rms + rtol * np.abs(expected)))


def within_contract_tolerance(actual, expected, out_dtype="bfloat16") -> bool:
    """ToleranceBound(atol 1e-2, rtol 1e-2) of aklr/ops/gemm/contract.py:203-209 with the output
    unit roundoff (bf16 2**-8, fp16 2**-11) added to rtol (aklr/core/contract/semantics/_compare.py:406-415)."""
    u = {"bfloat16": 2.0**-8, "float16": 2.0**-11}[out_dtype]
    atol, rtol = (1e-3, 1e-3) if out_dtype == "float16" else (1e-2, 1e-2)
    expected = np.asarray(expected, dtype=np.float64)
    err = np.abs(np.asarray(actual, dtype=np.float64) - expected)
    return bool(np.all(err <= atol + (rtol + u) * np.abs(expected)))


FP32_UNIT_ROUNDOFF = 2.0**-24
OUT_UNIT_ROUNDOFF = {"bfloat16": 2.0**-8, "float16": 2.0**-11}


def dot_product_bound(expected, magnitude, k: int, out_dtype="bfloat16", max_split_k=1) -> np.ndarray:
    """DotProductBound (aklr/core/contract/semantics/_compare.py:338-356), the gemm_a4w4_mxfp4 contract's
    error bound (aklr/ops/gemm/contract.py:375, max_split_k=1): per element
    B = 2 (6 sqrt(n_eff) + 2) u_fp32 * M + u_out * |y|, where M is the reference computed on the
    inputs' absolute values and n_eff = max over s <= max_split_k of ceil(k / s) + bit_length(s - 1)."""
    n_eff = max(-(-k // s) + (s - 1).bit_length() for s in range(1, max_split_k + 1))
    multiple = 6.0 * math.sqrt(n_eff) + 2.0
    return (2.0 * multiple * FP32_UNIT_ROUNDOFF * np.abs(np.asarray(magnitude, dtype=np.float64))
            + OUT_UNIT_ROUNDOFF[out_dtype] * np.abs(np.asarray(expected, dtype=np.float64)))


def within_dot_product_bound(actual, expected, magnitude, k: int, out_dtype="bfloat16", max_split_k=1) -> bool:
    """Every element within dot_product_bound (the gemm contracts compare with max_violation_fraction
    0, aklr/core/contract/spec/_args.py:203) and the errors unbiased: |mean| / rms <= 5 / sqrt(n)
    (ElementwiseBound's bias test, _compare.py:313-326)."""
    err = np.asarray(actual, dtype=np.float64) - np.asarray(expected, dtype=np.float64)
    if not np.all(np.abs(err) <= dot_product_bound(expected, magnitude, k, out_dtype, max_split_k)):
        return False
    rms = float(np.sqrt(np.mean(err * err))) if err.size else 0.0
    return rms == 0.0 or abs(float(err.mean())) / rms <= 5.0 / math.sqrt(err.size)

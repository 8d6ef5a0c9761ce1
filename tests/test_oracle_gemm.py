"""Pins oracle/gemm.py: a float64 element-by-element triple loop on tiny shapes (operands decoded by
torch's fp8 casts, scales looked up per element by block index); all-unit scales reduce to torch's
plain product of the decoded codes; K = 128 is one block; the partial last b_scale row; MN-major
a_scale equals K-major transposed; row/column sampling equals slicing; the MXFP4 product against a
literal e2m1 table with e8m0 exponents; and the tolerance checks reject a planted error."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gemm as g

E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def _codes(rng, shape, fmt=torch.float8_e4m3fn):
    x = torch.from_numpy(rng.standard_normal(shape).astype(np.float32) * 8)
    return x.to(fmt).view(torch.uint8).numpy()


def _dec(c, fmt=torch.float8_e4m3fn):
    return torch.from_numpy(c).view(fmt).double().numpy()


def _loop8(a, b, sa_k, sb, fmt=torch.float8_e4m3fn, bias=None):
    av, bv = _dec(a, fmt), _dec(b, fmt)
    m, k = a.shape
    n = b.shape[0]
    out = np.zeros((m, n))
    for i in range(m):
        for j in range(n):
            acc = 0.0
            for kk in range(k):
                acc += av[i, kk] * float(sa_k[i, kk // 128]) * bv[j, kk] * float(sb[j // 128, kk // 128])
            out[i, j] = acc + (0.0 if bias is None else float(bias[j]))
    return out


@pytest.mark.parametrize("fmt", [torch.float8_e4m3fn, torch.float8_e5m2])
def test_gemm8_triple_loop(fmt):
    rng = np.random.default_rng(0)
    m, n, k = 3, 144, 256  # n % 128 != 0: the last b_scale row covers 16 columns
    a, b = _codes(rng, (m, k), fmt), _codes(rng, (n, k), fmt)
    sa = np.exp2(rng.uniform(-3, 0, (m, k // 128))).astype(np.float32)
    sb = np.exp2(rng.uniform(-3, 0, (2, k // 128))).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    fname = "e4m3fn" if fmt == torch.float8_e4m3fn else "e5m2"
    got = g.gemm_a8w8_blockwise_scaled(a, b, sa, sb, fmt=fname, bias=bias)
    want = _loop8(a, b, sa, sb, fmt, bias)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-4 * np.abs(want).max())


def test_gemm8_unit_scales_is_plain_product_and_one_block():
    rng = np.random.default_rng(1)
    a, b = _codes(rng, (7, 128)), _codes(rng, (32, 128))
    ones_a, ones_b = np.ones((7, 1), np.float32), np.ones((1, 1), np.float32)
    got = g.gemm_a8w8_blockwise_scaled(a, b, ones_a, ones_b)
    want = (torch.from_numpy(a).view(torch.float8_e4m3fn).float() @
            torch.from_numpy(b).view(torch.float8_e4m3fn).float().T).numpy()
    assert np.allclose(got, want, rtol=1e-6)
    sa = np.full((7, 1), 0.5, np.float32)
    sb = np.full((1, 1), 0.25, np.float32)
    assert np.allclose(g.gemm_a8w8_blockwise_scaled(a, b, sa, sb), want * 0.125, rtol=1e-6)


def test_gemm8_mn_major_sampling_and_partial_block():
    rng = np.random.default_rng(2)
    m, n, k = 9, 272, 384
    a, b = _codes(rng, (m, k)), _codes(rng, (n, k))
    sa = rng.uniform(0.1, 1, (m, 3)).astype(np.float32)
    sb = rng.uniform(0.1, 1, (3, 3)).astype(np.float32)
    full = g.gemm_a8w8_blockwise_scaled(a, b, sa, sb)
    assert np.array_equal(full, g.gemm_a8w8_blockwise_scaled(a, b, np.ascontiguousarray(sa.T), sb,
                                                             scale_major_mode="MN"))
    r, c = np.array([0, 4, 8]), np.array([1, 130, 257, 271])
    sub = g.gemm_a8w8_blockwise_scaled(a, b, sa, sb, rows=r, cols=c)
    # same formula on the sampled operands; only BLAS's float32 summation order differs
    assert np.allclose(sub, full[np.ix_(r, c)], rtol=0, atol=1e-5 * np.sqrt(np.mean(full.astype(np.float64)**2)))
    # the last 16 columns use b_scale row 2: scaling that row alone scales only them
    sb2 = sb.copy()
    sb2[2] *= 2
    full2 = g.gemm_a8w8_blockwise_scaled(a, b, sa, sb2)
    assert np.allclose(full2[:, 256:], 2 * full[:, 256:], rtol=1e-6) and np.array_equal(full2[:, :256], full[:, :256])


def test_gemm4_against_literal_table():
    rng = np.random.default_rng(3)
    m, n, k = 3, 16, 128
    a = rng.integers(0, 256, (m, k // 2), dtype=np.uint8)
    b = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    sa = rng.integers(120, 135, (m, k // 32), dtype=np.uint8)
    sb = rng.integers(120, 135, (n, k // 32), dtype=np.uint8)
    want = np.zeros((m, n))
    for i in range(m):
        for j in range(n):
            for kk in range(k):
                byte_a, byte_b = a[i, kk // 2], b[j, kk // 2]
                na = byte_a & 15 if kk % 2 == 0 else byte_a >> 4
                nb = byte_b & 15 if kk % 2 == 0 else byte_b >> 4
                want[i, j] += (E2M1[na] * 2.0 ** (int(sa[i, kk // 32]) - 127)) * (
                    E2M1[nb] * 2.0 ** (int(sb[j, kk // 32]) - 127))
    bias = rng.standard_normal(n).astype(np.float32)
    got = g.gemm_a4w4_mxfp4(a, b, sa, sb, bias=bias)
    assert np.allclose(got, want + bias, rtol=1e-5, atol=1e-5 * np.abs(want).max())


def test_tolerance_checks_reject_planted_error():
    rng = np.random.default_rng(4)
    y = rng.standard_normal((64, 64)).astype(np.float32)
    assert g.within_north_star(y, y) and g.within_contract_tolerance(y, y)
    bad = y.copy()
    i = np.unravel_index(np.argmin(np.abs(y)), y.shape)
    bad[i] += 0.05 * np.sqrt(np.mean(y.astype(np.float64) ** 2))
    assert not g.within_north_star(bad, y)
    assert not g.within_contract_tolerance(bad, y)
    near = y * (1 + 2.0**-9)  # inside one bf16 rounding
    assert g.within_north_star(near, y) and g.within_contract_tolerance(near, y)


def test_dot_product_bound():
    # B = 2 (6 sqrt(k) + 2) 2**-24 M + 2**-8 |y| (the reference's DotProductBound, max_split_k 1);
    # k = 64 gives 100 * 2**-24 * M
    y = np.array([1.0, -2.0, 0.5, 3.0])
    mag = np.array([4.0, 4.0, 1.0, 8.0])
    b = g.dot_product_bound(y, mag, 64)
    np.testing.assert_allclose(b, 100 * 2.0**-24 * mag + 2.0**-8 * np.abs(y), rtol=1e-12)
    # splitting K never lengthens the effective reduction: k stays the largest term
    assert np.array_equal(g.dot_product_bound(y, mag, 8192, max_split_k=16), g.dot_product_bound(y, mag, 8192))
    rng = np.random.default_rng(0)
    y = rng.normal(size=4096)
    mag = np.abs(y) * 3 + 1
    bound = g.dot_product_bound(y, mag, 1024)
    sign = rng.choice([-1.0, 1.0], size=y.size)
    assert g.within_dot_product_bound(y + 0.5 * bound * sign, y, mag, 1024)  # inside, unbiased
    bad = y + 0.5 * bound * sign
    bad[17] = y[17] + 1.5 * bound[17]
    assert not g.within_dot_product_bound(bad, y, mag, 1024)  # one element outside
    assert not g.within_dot_product_bound(y + 0.5 * bound, y, mag, 1024)  # inside, but all one sign

"""Writes the golden fixtures of this directory (run from the repo root:
``python tests/golden/make_golden.py``).

Inputs are the reference's own small test Points (tests/ops/cases.py:469-525, :759-772 of AKLR),
seeded here, plus edge rows (zero groups, subnormals, ties, the bf16 maximum, outliers). Expected
outputs are computed WITHOUT the numpy oracle, so the fixtures pin it:

- quantizers: a torch-CPU restatement of the reference formulas (aklr/ops/quant/reference.py:9-48,
  aklr/ops/fused_moe/reference.py:21-37), whose float32 rounding is torch's own and whose e4m3fn
  rounding is torch's ``.to(torch.float8_e4m3fn)`` -- the library cast the reference calls;
- GEMMs: float64 products of the decoded operands, decoded with torch's fp8 casts and a literal
  e2m1 table, scales expanded element by element.

The reference itself is not imported or run. Each fixture is an ``.npz`` of inputs and outputs.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent
E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def bf16_input(rows: int, cols: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((rows, cols), generator=g)
    mask = torch.rand((rows, cols), generator=g) < 0.01
    x = torch.where(mask, x * 20.0, x)
    return x.to(torch.bfloat16)


def edge_rows(cols: int) -> torch.Tensor:
    """Three rows of edge cases, bf16."""
    x = torch.zeros((3, cols), dtype=torch.float32)
    # row 0: one huge value per 32-group, the rest small (ties around the amax-relative grid)
    for g0 in range(0, cols, 32):
        x[0, g0 : g0 + 32] = torch.linspace(-1.0, 1.0, 32) * (2.0 ** ((g0 // 32) % 7 - 3))
    x[0, 5] = 3.0e38
    # row 1: group 0 all zero (amax floor), group 1 bf16 subnormals, the rest exact binary fractions
    x[1, 128:256 if cols >= 256 else cols] = 1.0e-39
    x[1, 256:] = torch.arange(cols - 256).float() * 0.125 - 7.0 if cols > 256 else 0.0
    # row 2: values 448 * k / 64 (many exact e4m3 ties once divided by the group scale)
    x[2] = (torch.arange(cols).float() % 129 - 64.0) * 7.0
    return x.to(torch.bfloat16)


# ---------------------------------------------------------------------------------------------
def quant_fp8_torch(x: torch.Tensor):
    x = x.float()
    rows, cols = x.shape
    g = x.reshape(rows, cols // 128, 128)
    amax = g.abs().amax(-1).clamp_min(1e-10)
    scales = amax * (1.0 / 448.0)
    inv = 1.0 / scales
    v = (g * inv.unsqueeze(-1)).clamp(-448.0, 448.0)
    q = v.to(torch.float8_e4m3fn).reshape(rows, cols)
    return q.view(torch.uint8).numpy(), scales.t().contiguous().numpy()


def quant_mxfp8_torch(x: torch.Tensor):
    x = x.float()
    rows, cols = x.shape
    g = x.reshape(rows, cols // 32, 32)
    amax = g.abs().amax(-1).clamp_min(1e-10)
    raw = (amax * (1.0 / 448.0)).contiguous().view(torch.int32)
    e = (raw >> 23) + ((raw & 0x7FFFFF) != 0).to(torch.int32)
    scale = (e << 23).contiguous().view(torch.float32)
    v = (g / scale.unsqueeze(-1)).clamp(-448.0, 448.0)
    q = v.to(torch.float8_e4m3fn).reshape(rows, cols)
    return q.view(torch.uint8).numpy(), e.to(torch.uint8).numpy()


def quant_mxfp4_torch(x: torch.Tensor):
    """Codes by a brute-force nearest search over the 8 magnitudes (ties to the even code)."""
    x = x.float()
    rows, cols = x.shape
    g = x.reshape(rows, cols // 32, 32)
    amax = g.abs().amax(-1)
    finite = amax.isfinite()
    m, e = torch.frexp(torch.where(finite, amax, 0.0).clamp_min(1e-10))
    e = (e - 3 + (m > 0.75).int()).clamp(-127, 127)
    scaled = torch.where(finite.unsqueeze(-1), g, 0.0) / torch.exp2(e.float()).unsqueeze(-1)
    mags = torch.tensor(E2M1[:8])
    d = (scaled.abs().unsqueeze(-1) - mags).abs()  # [..., 8]
    best = torch.full(scaled.shape, -1, dtype=torch.int64)
    bestd = torch.full(scaled.shape, float("inf"))
    for i in range(8):
        better = (d[..., i] < bestd) | ((d[..., i] == bestd) & (i % 2 == 0))
        best = torch.where(better, i, best)
        bestd = torch.where(better, d[..., i], bestd)
    nib = best | ((scaled.view(torch.int32) < 0).long() << 3)
    nib = torch.where(finite.unsqueeze(-1), nib, 0).reshape(rows, cols)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).to(torch.uint8)
    sbytes = torch.where(finite, e + 127, 255).to(torch.uint8)
    return packed.numpy(), sbytes.numpy()


# ---------------------------------------------------------------------------------------------
def fp8_decode(codes: np.ndarray, fmt=torch.float8_e4m3fn) -> np.ndarray:
    return torch.from_numpy(codes).view(fmt).float().double().numpy()


def gemm8_f64(a, b, sa_k, sb):
    """a, b codes [m,k], [n,k]; sa_k [m, k/128]; sb [ceil(n/128), k/128]; float64 out."""
    av, bv = fp8_decode(a), fp8_decode(b)
    m, k = a.shape
    n = b.shape[0]
    out = np.zeros((m, n))
    for kb in range(k // 128):
        ks = slice(kb * 128, kb * 128 + 128)
        part = av[:, ks] @ bv[:, ks].T
        for j in range(n):
            out[:, j] += part[:, j] * sa_k[:, kb].astype(np.float64) * np.float64(sb[j // 128, kb])
    return out


def fp4_decode(packed: np.ndarray) -> np.ndarray:
    t = np.array(E2M1)
    lo, hi = packed & 15, packed >> 4
    v = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,))
    v[..., 0::2] = t[lo]
    v[..., 1::2] = t[hi]
    return v


def gemm4_f64(a, b, sa, sb):
    av, bv = fp4_decode(a), fp4_decode(b)
    ea = np.repeat(np.exp2(sa.astype(np.float64) - 127), 32, axis=1)
    eb = np.repeat(np.exp2(sb.astype(np.float64) - 127), 32, axis=1)
    return (av * ea) @ (bv * eb).T


def block_weight(n, k, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn((n, k), generator=g) * 0.02
    nb, kb = -(-n // 128), k // 128
    wp = torch.nn.functional.pad(w, (0, 0, 0, nb * 128 - n))
    blocks = wp.view(nb, 128, kb, 128)
    s = blocks.abs().amax(dim=(1, 3)).clamp_min(1e-10) / 448.0
    codes = (blocks / s[:, None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(nb * 128, k)[:n]
    return codes.contiguous().view(torch.uint8).numpy(), s.numpy()


def main() -> None:
    # quantizers: the reference's Point (3 x 256) as edge rows, and a seeded 16 x 1024
    for name, x in (("edge3x256", edge_rows(256)), ("seed16x1024", bf16_input(16, 1024, 7))):
        xb = x.view(torch.int16).numpy().view(np.uint16)
        q8, s8 = quant_fp8_torch(x)
        qm, sm = quant_mxfp8_torch(x)
        q4, s4 = quant_mxfp4_torch(x)
        np.savez_compressed(OUT / f"quant_{name}.npz", x_bf16_bits=xb, fp8_codes=q8, fp8_scales=s8,
                            mxfp8_codes=qm, mxfp8_scales=sm, mxfp4_packed=q4, mxfp4_scales=s4)

    # gemm_a8w8_blockwise_scaled: row_major m4 n16 k128 and b_shuffled m4 n128 k256 (cases.py:497-525),
    # plus m5 n144 k384 (a partial last b_scale row)
    for (m, n, k, seed) in ((4, 16, 128, 1), (4, 128, 256, 2), (5, 144, 384, 3)):
        x = bf16_input(m, k, seed)
        a, sa_gm = quant_fp8_torch(x)  # sa_gm: [k/128, m] group-major
        b, sb = block_weight(n, k, seed + 100)
        out = gemm8_f64(a, b, sa_gm.T, sb)
        np.savez_compressed(OUT / f"gemm8_m{m}_n{n}_k{k}.npz", a=a, a_scale_group_major=sa_gm, b=b, b_scale=sb,
                            out_f64=out)

    # gemm_a4w4_mxfp4: b_shuffled m4 n256 k256 (cases.py:469-482), plus m3 n32 k192 (K not a multiple of 128)
    for (m, n, k, seed) in ((4, 256, 256, 4), (3, 32, 192, 5)):
        a, sa = quant_mxfp4_torch(bf16_input(m, k, seed))
        g = torch.Generator().manual_seed(seed + 200)
        b, sb = quant_mxfp4_torch((torch.randn((n, k), generator=g) * 0.02).to(torch.bfloat16))
        np.savez_compressed(OUT / f"gemm4_m{m}_n{n}_k{k}.npz", a=a, a_scale=sa, b=b, b_scale=sb,
                            out_f64=gemm4_f64(a, b, sa, sb))
    print("wrote", sorted(p.name for p in OUT.glob("*.npz")))


if __name__ == "__main__":
    main()

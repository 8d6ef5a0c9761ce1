"""Seeded synthetic inputs of the benchmark configurations (torch, generated on any device).

The reference draws its inputs from the contracts' distributions (aklr/core/contract/semantics/
_workloads.py:54-95); the configurations measured here are stated as value distributions instead:

- activations: bf16 ~ N(0, 1), optionally with 1% of the entries multiplied by 20 (outliers);
- FP8 weights: fp32 ~ N(0, 0.02), quantized per 128x128 block to e4m3fn with s = amax / 448;
- MXFP4 weights: fp32 ~ N(0, 0.02), quantized per 1x32 along K to e2m1 with an e8m0 exponent
  (the same rule as the MXFP4 activation quantizer, aklr/ops/fused_moe/reference.py:21-37);
- MoE routing: per token, 8 distinct experts drawn with p(e) proportional to rank(e)^-1.1.
"""
from __future__ import annotations

import torch

DEEPSEEK_NK = ((2112, 7168), (24576, 1536), (7168, 16384))
LLAMA70B_NK = ((10240, 8192), (57344, 8192), (8192, 28672))
DECODE_M = (1, 4, 16, 64, 128)
PREFILL_M = (1024, 4096, 8192)
MXFP4_M = (1, 32, 512, 4096)


def generator(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def activations(m: int, k: int, *, seed: int = 0, device="cpu", outliers: bool = True) -> torch.Tensor:
    g = generator(seed, device)
    x = torch.randn((m, k), generator=g, device=device, dtype=torch.float32)
    if outliers:
        mask = torch.rand((m, k), generator=g, device=device) < 0.01
        x = torch.where(mask, x * 20.0, x)
    return x.to(torch.bfloat16)


def blockwise_fp8_weight(n: int, k: int, *, seed: int = 1, device="cpu", std: float = 0.02):
    """(e4m3fn codes [n, k], fp32 scales [ceil(n/128), k/128]); s = amax / 448 per 128x128 block
    (partial last row block when n % 128 != 0)."""
    g = generator(seed, device)
    w = torch.randn((n, k), generator=g, device=device, dtype=torch.float32) * std
    nb, kb = -(-n // 128), k // 128
    pad = nb * 128 - n
    wp = torch.nn.functional.pad(w, (0, 0, 0, pad)) if pad else w
    blocks = wp.view(nb, 128, kb, 128)
    amax = blocks.abs().amax(dim=(1, 3)).clamp_min(1e-10)
    scales = amax / 448.0
    codes = (blocks / scales[:, None, :, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    codes = codes.view(nb * 128, k)[:n].contiguous()
    return codes, scales.contiguous()


_E2M1_MIDPOINTS = (0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0)
_E2M1_TIE_UP = (False, True, False, True, False, True, False)  # a tie rounds to the even code


def mxfp4_quantize(x: torch.Tensor):
    """fp32/bf16 [r, k] -> (packed e2m1 uint8 [r, k/2], e8m0 bytes uint8 [r, k/32]); the MXFP4 rule
    of aklr/ops/fused_moe/reference.py:21-37, in torch (weights are prepared with it)."""
    x = x.float()
    r, k = x.shape
    blocks = x.view(r, k // 32, 32)
    amax = blocks.abs().amax(-1).clamp_min(1e-10)
    mant, expo = torch.frexp(amax)
    e = (expo - 3 + (mant > 0.75).int()).clamp(-127, 127)
    scaled = blocks / torch.exp2(e.float())[..., None]
    m = scaled.abs()
    idx = torch.zeros_like(m, dtype=torch.uint8)
    for mid, up in zip(_E2M1_MIDPOINTS, _E2M1_TIE_UP):
        idx += (m >= mid if up else m > mid).to(torch.uint8)
    sign = (scaled.view(torch.int32) < 0).to(torch.uint8) << 3  # the sign bit, -0 included
    nib = (idx | sign).view(r, k)
    packed = nib[:, 0::2] | (nib[:, 1::2] << 4)
    return packed.contiguous(), (e + 127).to(torch.uint8).contiguous()


def mxfp4_weight(n: int, k: int, *, seed: int = 1, device="cpu", std: float = 0.02):
    g = generator(seed, device)
    w = torch.randn((n, k), generator=g, device=device, dtype=torch.float32) * std
    return mxfp4_quantize(w)


def zipf_routing(tokens: int, experts: int = 256, top_k: int = 8, *, alpha: float = 1.1, seed: int = 3,
                 device="cpu") -> torch.Tensor:
    """[tokens, top_k] int64 expert ids, distinct per token, p(e) ~ (e + 1)^-alpha."""
    g = generator(seed, "cpu")
    p = torch.arange(1, experts + 1, dtype=torch.float64).pow(-alpha)
    ids = torch.multinomial(p.expand(tokens, experts), top_k, replacement=False, generator=g)
    return ids.to(device)


def moe_expert_weights(experts: int, rows: int, cols: int, *, seed: int = 1, device="cpu", std: float = 0.02):
    """Stacked expert weights of the MoE configuration: per expert, fp32 ~ N(0, std) [rows, cols]
    quantized per 128x128 block to e4m3fn with s = amax / 448, as blockwise_fp8_weight. Returns (codes
    e4m3fn [experts, rows, cols], fp32 scales [experts, ceil(rows/128), cols/128]); expert e draws from
    seed + e."""
    codes = torch.empty((experts, rows, cols), dtype=torch.float8_e4m3fn, device=device)
    scales = torch.empty((experts, -(-rows // 128), cols // 128), dtype=torch.float32, device=device)
    for e in range(experts):
        c, s = blockwise_fp8_weight(rows, cols, seed=seed + e, device=device, std=std)
        codes[e].copy_(c)
        scales[e].copy_(s)
    return codes, scales


def moe_routing(tokens: int, experts: int = 256, top_k: int = 8, *, seed: int = 3, device="cpu"):
    """Config-5 routing as the experts take it: Zipf(1.1) ids [tokens, top_k] plus the shared expert
    (id ``experts``) in the last slot, int32; weights fp32 [tokens, top_k + 1] ~ U(0, 1), the shared
    slot at 1."""
    ids = zipf_routing(tokens, experts, top_k, seed=seed, device="cpu").to(torch.int32)
    ids = torch.cat([ids, torch.full((tokens, 1), experts, dtype=torch.int32)], 1)
    g = generator(seed + 1, "cpu")
    wts = torch.rand((tokens, top_k + 1), generator=g)
    wts[:, -1] = 1.0
    return ids.to(device), wts.to(device)

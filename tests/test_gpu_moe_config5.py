"""GPU parity of the grouped DeepSeek FP8 MoE at config 5's model dimensions (
DeepSeek-V3 experts, model_dim 7168, inter_dim 2048 -- gate_up N=4096, K=7168 (56 K blocks), down
N=7168, K=2048 (16 K blocks) -- top-8 routing with Zipf(1.1)-skewed expert counts, the shared expert
last at weight 1).

- The experts against the oracle (oracle/moe.py) at SQNR >= 30 dB (the contract's SqnrBound,
  aklr/plugins/sglang/models/deepseek_v2/contract.py:300-306), with as many experts as the host oracle
  computes in seconds (16-32 routed), both weight layouts, and token counts whose per-expert row counts
  cover the 64-, 128- and 256-row block classes (and full 256-row blocks with remainders).
- The whole op (router, grouped top-k, experts) at the same dimensions, with router inputs whose
  products are exact in fp32 so both sides route alike.
- The full config-5 call (256 routed experts, T = 64 and T = 4096, 257 expert slots, Zipf(1.1) routing,
  the 610 MiB workspace layout at T = 4096) by two properties: relabelling the routed experts (weights,
  scales and ids permuted together) leaves the output bit-identical, and sampled tokens match the oracle
  computed from only those tokens' experts, copied to the host.
- The whole op at 256 routed experts with grouped top-k (8 groups, 4 kept) on router inputs whose
  products are exact in fp32: sampled tokens against the oracle's routing (computed for every token on
  the host) and their experts.
- A call past the kernels' per-call token limit (32-bit offsets: 16644 tokens at 9 slots of 7168) runs
  as consecutive calls: its rows equal, bit for bit, a call on those rows alone.

The full-size calls draw BASELINE's weights: N(0, 0.02) per expert, block-quantized per 128 x 128 to
e4m3fn with s = amax / 448 (workloads.moe_expert_weights). The smaller checks draw N(0, 64) cast to
e4m3fn (within +-448, as the contract's finite fp8 draws) with 128 x 128 block scales log-uniform in
[2**-3, 1] / 512, which spreads the scales over the fold's exponent range.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import aklr_amd
from aklr_amd import layouts, workloads
from oracle import formats, moe
from tests.helpers import bf16_bits, f32, say, u8

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
D, INTER, TOPK = 7168, 2048, 8


def _weights(n_experts, seed, d=D, inter=INTER):
    """e4m3fn w1 [E, 2I, D], w2 [E, D, I] and fp32 block scales, drawn on the GPU one expert at a time."""
    g = workloads.generator(seed, DEV)
    w1 = torch.empty((n_experts, 2 * inter, d), dtype=torch.float8_e4m3fn, device=DEV)
    w2 = torch.empty((n_experts, d, inter), dtype=torch.float8_e4m3fn, device=DEV)
    for e in range(n_experts):
        w1[e] = (torch.randn((2 * inter, d), device=DEV, generator=g) * 64.0).to(torch.float8_e4m3fn)
        w2[e] = (torch.randn((d, inter), device=DEV, generator=g) * 64.0).to(torch.float8_e4m3fn)
    s1 = torch.exp2(torch.rand((n_experts, 2 * inter // 128, d // 128), device=DEV, generator=g) * 3 - 3) / 512
    s2 = torch.exp2(torch.rand((n_experts, d // 128, inter // 128), device=DEV, generator=g) * 3 - 3) / 512
    return w1, s1, w2, s2


def _zipf(t, n_routed, seed):
    """Zipf(1.1) routing, 8 distinct routed experts per token, plus the shared slot; weights U(0.05, 0.5)."""
    ids = workloads.zipf_routing(t, n_routed, TOPK, alpha=1.1, seed=seed).to(torch.int32)
    ids = torch.cat([ids, torch.full((t, 1), n_routed, dtype=torch.int32)], 1)
    g = workloads.generator(seed + 1, "cpu")
    w = (torch.rand((t, TOPK + 1), generator=g) * 0.45 + 0.05).float()
    w[:, TOPK] = 1.0
    return ids.numpy(), w.numpy()


def _host(*ts):
    return [u8(t) if t.dtype == torch.float8_e4m3fn else f32(t) for t in ts]


def _block_classes(ids, n_experts):
    """The row-block classes the kernels use for these per-expert counts: full 256-row blocks, then a
    remainder of the smallest of 64, 128, 256 that holds it."""
    counts = np.bincount(ids[(ids >= 0) & (ids < n_experts)], minlength=n_experts)
    classes = set()
    for c in counts[counts > 0]:
        if c >= 256:
            classes.add("256-full")
        r = c % 256
        if r:
            classes.add(64 if r <= 64 else (128 if r <= 128 else 256))
    return classes


@pytest.mark.parametrize("shuffled", [False, True])
@pytest.mark.parametrize("t,n_routed", [(64, 32), (320, 16)])
def test_experts_at_config5_dims(t, n_routed, shuffled):
    say(f"moe experts config-5 dims t={t} n_routed={n_routed} shuffled={shuffled}")
    w1, s1, w2, s2 = _weights(n_routed + 1, seed=t + n_routed)
    x = workloads.activations(t, D, seed=t, device=DEV, outliers=False)
    ids, w = _zipf(t, n_routed, seed=t)
    classes = _block_classes(ids, n_routed + 1)
    # t = 64: every expert in the 64-row class; t = 320: full blocks and all three remainder classes
    assert classes == ({64} if t == 64 else {64, 128, 256, "256-full"}), classes
    tw1, tw2 = (layouts.shuffle_weight(w1), layouts.shuffle_weight(w2)) if shuffled else (w1, w2)
    out = aklr_amd.moe_fp8_experts(x, tw1, tw2, torch.from_numpy(w).to(DEV), torch.from_numpy(ids).to(DEV), s1, s2)
    torch.cuda.synchronize()
    hw1, hs1, hw2, hs2 = _host(w1, s1, w2, s2)
    ref = moe.moe_experts(f32(x), ids, w, hw1, hs1, hw2, hs2)
    q = moe.sqnr_db(formats.round_to_bf16(ref), f32(out))
    say(f"  sqnr {q:.1f} dB")
    assert q >= 30.0


def test_deepseek_v2_fp8_moe_at_config5_dims():
    t, n_routed, g, tg = 32, 32, 8, 4
    say(f"deepseek_v2_fp8_moe config-5 dims t={t} n_routed={n_routed}")
    rng = np.random.default_rng(55)
    # router products exact in fp32: hidden in multiples of 1/16 within [-1, 1], router weights in
    # {-1, 0, 1}/16 (a sum of 7168 such products needs at most 17 bits)
    x = (rng.integers(-16, 17, size=(t, D)) / 16.0).astype(np.float32)
    wr = (rng.integers(-1, 2, size=(n_routed, D)) / 16.0).astype(np.float32)
    bias = formats.round_to_bf16(rng.normal(scale=0.02, size=n_routed).astype(np.float32))
    w1, s1, w2, s2 = _weights(n_routed + 1, seed=56)
    tw1, tw2 = layouts.shuffle_weight(w1), layouts.shuffle_weight(w2)
    xb = torch.from_numpy(x).to(DEV).to(torch.bfloat16)
    out = aklr_amd.deepseek_v2_fp8_moe(xb, torch.from_numpy(wr).to(DEV).to(torch.bfloat16),
                                       torch.from_numpy(bias).to(DEV).to(torch.bfloat16), tw1, s1, tw2, s2, TOPK, g, tg,
                                       True, "sigmoid", 2.5)
    assert isinstance(out, torch.Tensor), out
    torch.cuda.synchronize()
    hw1, hs1, hw2, hs2 = _host(w1, s1, w2, s2)
    ref = moe.deepseek_v2_fp8_moe(x, wr, bias, hw1, hs1, hw2, hs2, TOPK, g, tg, True, 2.5)
    q = moe.sqnr_db(formats.round_to_bf16(ref), f32(out))
    say(f"  sqnr {q:.1f} dB")
    assert q >= 30.0


def _baseline_weights(n_experts, seed):
    """BASELINE configs[4]'s expert weights: N(0, 0.02), 128 x 128 block-quantized to e4m3fn."""
    w1, s1 = workloads.moe_expert_weights(n_experts, 2 * INTER, D, seed=seed, device=DEV)
    w2, s2 = workloads.moe_expert_weights(n_experts, D, INTER, seed=seed + 1000, device=DEV)
    return w1, s1, w2, s2


def _sampled_reference(toks, x, ids, w, w1, s1, w2, s2):
    """The oracle output of tokens ``toks`` from only their own experts (host copies of those)."""
    xs = f32(x[toks])
    ref = np.zeros_like(xs)
    for e in np.unique(ids[toks]).tolist():
        hw1, hs1, hw2, hs2 = _host(w1[e], s1[e], w2[e], s2[e])
        rows, slots = np.nonzero(ids[toks] == e)
        y = moe.expert_mlp(xs[rows], hw1, hs1, hw2, hs2)
        np.add.at(ref, rows, w[toks][rows, slots][:, None] * y)
    return ref


@pytest.mark.parametrize("t", [64, 4096])
def test_config5_full_call_relabel_and_sampled_tokens(t):
    n_routed = 256
    say(f"moe config 5 full call t={t} n_routed={n_routed}")
    w1, s1, w2, s2 = _baseline_weights(n_routed + 1, seed=5)
    x = workloads.activations(t, D, seed=6, device=DEV, outliers=False)
    ids, w = _zipf(t, n_routed, seed=7)
    tids, tw = torch.from_numpy(ids).to(DEV), torch.from_numpy(w).to(DEV)
    out = aklr_amd.moe_fp8_experts(x, w1, w2, tw, tids, s1, s2)
    torch.cuda.synchronize()
    assert not torch.isnan(out.float()).any()
    # relabel: routed expert e becomes perm[e] (weights, scales and ids together); the shared one stays last
    perm = torch.randperm(n_routed, generator=workloads.generator(8, "cpu")).to(DEV)
    full = torch.cat([perm, torch.tensor([n_routed], device=DEV)])
    say("  relabelled call")
    pw1, ps1, pw2, ps2 = (torch.empty_like(a) for a in (w1, s1, w2, s2))
    for src, dst in ((w1, pw1), (s1, ps1), (w2, pw2), (s2, ps2)):
        bytes_of = (lambda a: a.view(torch.uint8)) if src.dtype == torch.float8_e4m3fn else (lambda a: a)
        bytes_of(dst).index_copy_(0, full, bytes_of(src))
    out_p = aklr_amd.moe_fp8_experts(x, pw1, pw2, tw, full[tids.long()].to(torch.int32), ps1, ps2)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out_p.view(torch.int16)), "relabelling the experts changed the output"
    del pw1, ps1, pw2, ps2
    # sampled tokens against the oracle, from their own <= 9 experts each
    toks = [0, 1234, 2047, 4095] if t == 4096 else [0, 21, 42, 63]
    ref = _sampled_reference(toks, x, ids, w, w1, s1, w2, s2)
    q = moe.sqnr_db(formats.round_to_bf16(ref), f32(out[toks]))
    say(f"  sampled tokens sqnr {q:.1f} dB")
    assert q >= 30.0


def test_deepseek_v2_fp8_moe_full_router_sampled_tokens():
    # the whole op at config 5's expert count: router over 256 experts, grouped top-k (8 groups, 4 kept),
    # renormalized weights x 2.5, the shared expert last; router products exact in fp32 (hidden in
    # multiples of 1/16 within [-1, 1], router weights in {-1, 0, 1}/16), so GPU and host route alike
    t, n_routed, g, tg = 64, 256, 8, 4
    say(f"deepseek_v2_fp8_moe full router t={t} n_routed={n_routed}")
    rng = np.random.default_rng(57)
    x = (rng.integers(-16, 17, size=(t, D)) / 16.0).astype(np.float32)
    wr = (rng.integers(-1, 2, size=(n_routed, D)) / 16.0).astype(np.float32)
    bias = formats.round_to_bf16(rng.normal(scale=0.02, size=n_routed).astype(np.float32))
    w1, s1, w2, s2 = _baseline_weights(n_routed + 1, seed=58)
    xb = torch.from_numpy(x).to(DEV).to(torch.bfloat16)
    out = aklr_amd.deepseek_v2_fp8_moe(xb, torch.from_numpy(wr).to(DEV).to(torch.bfloat16),
                                       torch.from_numpy(bias).to(DEV).to(torch.bfloat16), w1, s1, w2, s2, TOPK, g, tg,
                                       True, "sigmoid", 2.5)
    assert isinstance(out, torch.Tensor), out
    torch.cuda.synchronize()
    logits = moe.router_logits(x, wr)
    ids, wts = moe.grouped_topk(logits, bias, TOPK, g, tg, True, 2.5)
    ids, wts = moe.with_shared_slot(ids, wts, n_routed)
    assert len(np.unique(ids[:, :TOPK])) > 64, "the routing touches a small part of the experts"
    toks = [0, 17, 38, 63]
    ref = _sampled_reference(toks, xb, ids, wts, w1, s1, w2, s2)
    q = moe.sqnr_db(formats.round_to_bf16(ref), f32(out[toks]))
    say(f"  sampled tokens sqnr {q:.1f} dB")
    assert q >= 30.0


def test_call_past_the_per_call_token_limit_runs_in_chunks():
    # 8 routed experts, all picked by every token, plus the shared one: 9 slots of 7168, so one library
    # call takes at most 16644 tokens; 17000 runs as two. Every token's output depends on that token alone,
    # so rows at the start, across the chunk boundary and at the end equal a call on those rows alone.
    t, n_routed, inter = 17000, 8, 256
    say(f"moe experts chunked t={t}")
    w1, s1, w2, s2 = _weights(n_routed + 1, seed=9, inter=inter)
    x = workloads.activations(t, D, seed=10, device=DEV, outliers=False)
    ids = torch.arange(n_routed + 1, dtype=torch.int32, device=DEV).repeat(t, 1)
    w = torch.rand((t, n_routed + 1), device=DEV, generator=workloads.generator(11, DEV))
    from aklr_amd import moe as hm

    assert len(hm.token_chunks(t, D, inter, n_routed + 1)) == 2
    out = aklr_amd.moe_fp8_experts(x, w1, w2, w, ids, s1, s2)
    rows = torch.cat([torch.arange(0, 8), torch.arange(16640, 16648), torch.arange(t - 8, t)]).to(DEV)
    part = aklr_amd.moe_fp8_experts(x[rows], w1, w2, w[rows], ids[rows], s1, s2)
    torch.cuda.synchronize()
    assert torch.equal(out[rows].view(torch.int16), part.view(torch.int16))

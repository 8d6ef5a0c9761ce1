"""GPU parity of the grouped DeepSeek FP8 MoE (aklr_moe_fp8_route / _experts / aklr_deepseek_v2_fp8_moe)
against the CPU oracle (oracle/moe.py).

Bounds, written here:
- routing: ids bit-exact against the oracle's grouped top-k on the same bf16 logits, except on tokens
  whose decision is a near-tie (the competing biased scores within 1e-6 relative; sigmoid rounding
  may differ by an ulp between implementations); such tokens must be under 5% of the total.
  Weights within rtol 1e-5.
- outputs: SQNR >= 30 dB against the oracle's output rounded to bf16 -- the contract's SqnrBound
  (aklr/plugins/sglang/models/deepseek_v2/contract.py:300-306). The full op is fed inputs whose router
  products are exact in fp32 (small dyadic values), so both sides route identically.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import aklr_amd
from aklr_amd import layouts
from oracle import formats, moe
from tests.helpers import bf16_bits, f32, say

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(formats.f32_to_bf16_bits(a.astype(np.float32)).view(np.int16)).view(torch.bfloat16).to(DEV)


def _experts(rng, e, inter, d):
    """fp8 expert weights with 128x128 block scales log-uniform in [2**-3, 1] (contract.py:251)."""
    w1 = formats.f32_to_e4m3fn(rng.normal(scale=64.0, size=(e, 2 * inter, d)).astype(np.float32))
    w2 = formats.f32_to_e4m3fn(rng.normal(scale=64.0, size=(e, d, inter)).astype(np.float32))
    s1 = (2.0 ** rng.uniform(-3, 0, size=(e, 2 * inter // 128, d // 128)) / 512).astype(np.float32)
    s2 = (2.0 ** rng.uniform(-3, 0, size=(e, d // 128, inter // 128)) / 512).astype(np.float32)
    return w1, s1, w2, s2


def _dev_weights(w1, s1, w2, s2, shuffled):
    t1 = torch.from_numpy(w1).view(torch.float8_e4m3fn).to(DEV)
    t2 = torch.from_numpy(w2).view(torch.float8_e4m3fn).to(DEV)
    if shuffled:
        t1, t2 = layouts.shuffle_weight(t1), layouts.shuffle_weight(t2)
    return t1, torch.from_numpy(s1).to(DEV), t2, torch.from_numpy(s2).to(DEV)


def _sqnr(out: torch.Tensor, ref: np.ndarray) -> float:
    return moe.sqnr_db(formats.round_to_bf16(ref), f32(out))


def _routing_tie(biased_row, topk, g, tg, tol=1e-6):
    """Whether this token's routing sits on a near-tie that an ulp of the sigmoid could flip: the
    topk_group-th and next group scores (a group scored by its two best biased scores), or, within the
    kept groups, the topk-th and next biased scores. Values within ``tol`` relative count as tied."""
    close = lambda a, b: abs(a - b) <= tol * max(abs(a), abs(b), 1e-30)
    e = biased_row.size
    per = e // g
    cand = np.arange(e)
    if g > 1:
        gs = np.sort(biased_row.reshape(g, per), axis=-1)[:, -2:].sum(-1, dtype=np.float32)
        srt = np.sort(gs)[::-1]
        if tg < g and close(srt[tg - 1], srt[tg]):
            return True
        kept = np.sort(np.argsort(-gs, kind="stable")[:tg])
        cand = np.concatenate([np.arange(k * per, (k + 1) * per) for k in kept])
    vals = np.sort(biased_row[cand])[::-1]
    return len(vals) > topk and close(vals[topk - 1], vals[topk])


@pytest.mark.parametrize("e,g,tg,topk,t", [(256, 8, 4, 8, 300), (64, 1, 1, 6, 97), (16, 8, 4, 8, 33)])
def test_route_matches_oracle(e, g, tg, topk, t):
    say(f"moe route e={e} g={g} tg={tg} topk={topk} t={t}")
    rng = np.random.default_rng(e + t)
    logits = formats.round_to_bf16(rng.normal(scale=2.0, size=(t, e)).astype(np.float32))
    bias = formats.round_to_bf16(rng.normal(scale=0.05, size=e).astype(np.float32))
    ids, w = aklr_amd.moe_fp8_route(_bf16(logits), _bf16(bias), topk, g, tg, True, 2.5, append_shared=True)
    torch.cuda.synchronize()
    ids_w, w_w = moe.grouped_topk(logits, bias, topk, g, tg, True, 2.5)
    ids_w, w_w = moe.with_shared_slot(ids_w, w_w, e)
    got_ids, got_w = ids.cpu().numpy(), w.cpu().numpy()
    biased = (moe.sigmoid32(logits) + bias).astype(np.float32)
    ties = 0
    for i in range(t):
        if np.array_equal(got_ids[i], ids_w[i]):
            np.testing.assert_allclose(got_w[i], w_w[i], rtol=1e-5)
            continue
        if set(got_ids[i, :topk].tolist()) == set(ids_w[i, :topk].tolist()):
            # the same picks in another order: only between picks whose biased scores are (near-)equal,
            # each pick keeping its weight
            np.testing.assert_allclose(biased[i][got_ids[i, :topk]], biased[i][ids_w[i, :topk]], rtol=1e-6)
            by_id = dict(zip(ids_w[i].tolist(), w_w[i].tolist()))
            np.testing.assert_allclose(got_w[i], [by_id[j] for j in got_ids[i].tolist()], rtol=1e-5)
        else:
            assert _routing_tie(biased[i], topk, g, tg), f"token {i}: {got_ids[i]} != {ids_w[i]} without a tie"
        ties += 1
    assert ties <= 0.05 * t
    assert np.all(got_ids[:, topk] == e) and np.all(got_w[:, topk] == 1.0)


def test_route_ties_take_lower_index():
    say("moe route ties")
    logits = np.zeros((4, 64), np.float32)
    ids, w = aklr_amd.moe_fp8_route(_bf16(logits), _bf16(np.zeros(64, np.float32)), 8, 8, 4, True, 2.5)
    want, _ = moe.grouped_topk(logits, np.zeros(64, np.float32), 8, 8, 4, True, 2.5)
    assert np.array_equal(ids.cpu().numpy()[:, :8], want)
    np.testing.assert_allclose(w.cpu().numpy()[:, :8], 2.5 / 8, rtol=1e-6)


def _zipf_routing(rng, t, n_routed, topk):
    p = 1.0 / np.arange(1, n_routed + 1) ** 1.1
    p /= p.sum()
    ids = np.stack([rng.choice(n_routed, topk, replace=False, p=p) for _ in range(t)]).astype(np.int32)
    w = rng.uniform(0.05, 0.5, size=(t, topk)).astype(np.float32)
    return moe.with_shared_slot(ids, w, n_routed)


@pytest.mark.parametrize("shuffled", [False, True])
@pytest.mark.parametrize("t,n_routed,d,inter", [(1, 16, 256, 256), (40, 16, 256, 128), (130, 8, 384, 384),
                                                  (300, 4, 256, 128), (700, 8, 256, 256)])
def test_experts_match_oracle(t, n_routed, d, inter, shuffled):
    say(f"moe experts t={t} n_routed={n_routed} d={d} inter={inter} shuffled={shuffled}")
    rng = np.random.default_rng(t * 7 + d)
    w1, s1, w2, s2 = _experts(rng, n_routed + 1, inter, d)
    x = formats.round_to_bf16(rng.normal(size=(t, d)).astype(np.float32))
    ids, w = _zipf_routing(rng, t, n_routed, min(8, n_routed))  # >= 256 rows per busy expert at t >= 300
    tw1, ts1, tw2, ts2 = _dev_weights(w1, s1, w2, s2, shuffled)
    out = aklr_amd.moe_fp8_experts(_bf16(x), tw1, tw2, torch.from_numpy(w).to(DEV), torch.from_numpy(ids).to(DEV),
                                   ts1, ts2)
    torch.cuda.synchronize()
    ref = moe.moe_experts(x, ids, w, w1, s1, w2, s2)
    q = _sqnr(out, ref)
    say(f"  sqnr {q:.1f} dB")
    assert q >= 30.0


def test_experts_skip_invalid_ids_and_are_deterministic():
    say("moe experts invalid ids / determinism")
    rng = np.random.default_rng(5)
    e, d, inter, t = 9, 256, 256, 24
    w1, s1, w2, s2 = _experts(rng, e, inter, d)
    x = formats.round_to_bf16(rng.normal(size=(t, d)).astype(np.float32))
    ids, w = _zipf_routing(rng, t, e - 1, 4)
    ids[::3, 1] = -1
    ids[1::5, 2] = e  # past the experts
    tw = _dev_weights(w1, s1, w2, s2, False)
    args = (_bf16(x), tw[0], tw[2], torch.from_numpy(w).to(DEV), torch.from_numpy(ids).to(DEV), tw[1], tw[3])
    out1 = aklr_amd.moe_fp8_experts(*args)
    out2 = aklr_amd.moe_fp8_experts(*args)
    torch.cuda.synchronize()
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16))
    keep = (ids >= 0) & (ids < e)
    ref = moe.moe_experts(x, np.where(keep, ids, 0), np.where(keep, w, 0.0).astype(np.float32), w1, s1, w2, s2)
    assert _sqnr(out1, ref) >= 30.0


@pytest.mark.parametrize("shuffled", [False, True])
@pytest.mark.parametrize("t,n_routed,g,tg,d,inter", [(1, 16, 8, 4, 256, 256), (64, 32, 8, 4, 256, 128),
                                                    (17, 24, 1, 1, 384, 256), (400, 16, 8, 4, 256, 128)])
def test_deepseek_v2_fp8_moe_matches_oracle(t, n_routed, g, tg, d, inter, shuffled):
    say(f"deepseek_v2_fp8_moe t={t} n_routed={n_routed} g={g} tg={tg} d={d} inter={inter} shuffled={shuffled}")
    rng = np.random.default_rng(t + n_routed + d)
    # router products exact in fp32: hidden in multiples of 1/16 within [-1, 1], router weights in
    # {-1, 0, 1}/16, so GPU and oracle logits are the same fp32 value before the bf16 rounding
    x = (rng.integers(-16, 17, size=(t, d)) / 16.0).astype(np.float32)
    wr = (rng.integers(-1, 2, size=(n_routed, d)) / 16.0).astype(np.float32)
    bias = formats.round_to_bf16(rng.normal(scale=0.02, size=n_routed).astype(np.float32))
    w1, s1, w2, s2 = _experts(rng, n_routed + 1, inter, d)
    tw1, ts1, tw2, ts2 = _dev_weights(w1, s1, w2, s2, shuffled)
    out = aklr_amd.deepseek_v2_fp8_moe(_bf16(x), _bf16(wr), _bf16(bias), tw1, ts1, tw2, ts2, 8, g, tg, True,
                                       "sigmoid", 2.5)
    assert isinstance(out, torch.Tensor), out
    torch.cuda.synchronize()
    ref = moe.deepseek_v2_fp8_moe(x, wr, bias, w1, s1, w2, s2, 8, g, tg, True, 2.5)
    q = _sqnr(out, ref)
    say(f"  sqnr {q:.1f} dB")
    assert q >= 30.0
    info = aklr_amd.deepseek_v2_fp8_moe.serving(_bf16(x), _bf16(wr), _bf16(bias), tw1, ts1, tw2, ts2, 8, g, tg, True,
                                                "sigmoid", 2.5)
    assert info.variant == ("shuffled_16x16" if shuffled else "row_major")

"""Pins for oracle/moe.py (the grouped DeepSeek FP8 MoE restatement). Each check is chosen so a
plausible mistake (biased weights, a group scored by one expert, ties resolved upward, the a1
multiply in place of the division, gate/up swapped, the shared slot dropped) fails it."""
import numpy as np
import pytest

from oracle import formats, gemm as ogemm, moe, quant as oquant


def _rng(seed=0):
    return np.random.default_rng(seed)


def test_ungrouped_routing_is_plain_topk():
    rng = _rng(1)
    logits = formats.round_to_bf16(rng.normal(size=(32, 64)).astype(np.float32))
    bias = rng.normal(scale=0.1, size=64).astype(np.float32)
    ids, w = moe.grouped_topk(logits, bias, 6, 1, 1, False, 1.0)
    biased = 1.0 / (1.0 + np.exp(-logits.astype(np.float64))) + bias
    for t in range(32):
        want = np.argpartition(-biased[t], 6)[:6]
        assert set(ids[t].tolist()) == set(want.tolist())
        assert np.all(np.diff(biased[t][ids[t]]) <= 0)  # descending


def test_grouped_routing_invariants():
    rng = _rng(2)
    e, g, tg, k = 64, 8, 3, 6
    logits = formats.round_to_bf16(rng.normal(size=(40, e)).astype(np.float32))
    bias = rng.normal(scale=0.2, size=e).astype(np.float32)
    ids, _ = moe.grouped_topk(logits, bias, k, g, tg, True, 2.5)
    biased = (moe.sigmoid32(logits) + bias).astype(np.float32)
    per = e // g
    for t in range(40):
        gs = np.sort(biased[t].reshape(g, per), axis=-1)[:, -2:].sum(-1)
        kept = set(np.argsort(-gs, kind="stable")[:tg].tolist())
        assert {int(i) // per for i in ids[t]} <= kept
        allowed = [i for i in range(e) if i // per in kept]
        rest = [i for i in allowed if i not in set(ids[t].tolist())]
        assert biased[t][ids[t]].min() >= max(biased[t][rest])


def test_group_score_sums_two_best():
    # group 0: one very high expert; group 1: two good ones whose sum beats group 0's top-2
    logits = np.full((1, 8), -8.0, dtype=np.float32)
    logits[0, 0] = 8.0                     # group 0 = experts 0..3
    logits[0, 4] = logits[0, 5] = 3.0      # group 1 = experts 4..7
    ids, _ = moe.grouped_topk(formats.round_to_bf16(logits), np.zeros(8, np.float32), 2, 2, 1, False, 1.0)
    assert sorted(ids[0].tolist()) == [4, 5]  # one-best scoring would keep group 0


def test_ties_lower_index_first():
    logits = np.zeros((1, 16), dtype=np.float32)
    ids, _ = moe.grouped_topk(logits, np.zeros(16, np.float32), 4, 4, 2, False, 1.0)
    assert ids[0].tolist() == [0, 1, 2, 3]


def test_weights_are_unbiased_scores_renormalized_and_scaled():
    rng = _rng(3)
    logits = formats.round_to_bf16(rng.normal(size=(8, 32)).astype(np.float32))
    bias = np.zeros(32, np.float32)
    bias[31] = 100.0  # forces expert 31 into every pick, its weight still its unbiased score
    ids, w = moe.grouped_topk(logits, bias, 4, 1, 1, True, 2.5)
    assert np.all(ids[:, 0] == 31)
    s = moe.sigmoid32(logits)
    raw = np.take_along_axis(s, ids, axis=-1)
    np.testing.assert_allclose(w, raw / raw.sum(-1, keepdims=True) * 2.5, rtol=1e-6)
    np.testing.assert_allclose(w.sum(-1), 2.5, rtol=1e-6)


def test_fp8_input_scale_is_a_division():
    # find amax values whose amax/448 and amax*fl32(1/448) differ in fp32
    vals = np.float32(1.0) + np.arange(1, 4000, dtype=np.float32) * np.float32(2**-12)
    div = (vals / np.float32(448.0)).astype(np.float32)
    mul = (vals * oquant.INV448).astype(np.float32)
    diff = np.nonzero(div != mul)[0]
    assert diff.size > 0
    amax = vals[diff[0]]
    x = np.zeros((1, 128), np.float32)
    x[0, 0] = amax
    x[0, 1:] = formats.round_to_bf16(np.linspace(-1, 1, 127, dtype=np.float32))
    x = formats.round_to_bf16(x)
    q, s = moe.quant_fp8_div(x)
    assert s[0, 0] == (formats.round_to_bf16(np.array([amax]))[0] / np.float32(448.0)).astype(np.float32)
    assert formats.fp8_to_f32(q[:, :1])[0, 0] == 448.0
    # dequant within half an e4m3 ulp (2**-3 relative for normals) of the bf16 input
    deq = formats.fp8_to_f32(q) * s[0, 0]
    assert np.all(np.abs(deq - x) <= np.abs(x) * 2**-4 + s[0, 0] * 2**-10)


def test_all_zero_group_uses_tiny_scale():
    q, s = moe.quant_fp8_div(np.zeros((2, 256), np.float32))
    assert np.all(q == 0) and np.all(s == np.finfo(np.float32).tiny)


def test_fp8_linear_reduces_to_a8w8_gemm():
    rng = _rng(4)
    x = rng.normal(size=(5, 256)).astype(np.float32)
    w = formats.f32_to_e4m3fn(rng.normal(scale=30, size=(144, 256)).astype(np.float32))
    ws = rng.uniform(0.01, 0.1, size=(2, 2)).astype(np.float32)
    q, s = moe.quant_fp8_div(x)
    want = ogemm.gemm_a8w8_blockwise_scaled(q, w, s, ws)
    np.testing.assert_allclose(moe.fp8_linear(x, w, ws), want, rtol=1e-5, atol=1e-5)


def _weights(rng, e, inter, d):
    w1 = formats.f32_to_e4m3fn(rng.normal(scale=40, size=(e, 2 * inter, d)).astype(np.float32))
    s1 = rng.uniform(2**-9, 2**-7, size=(e, 2 * inter // 128, d // 128)).astype(np.float32)
    w2 = formats.f32_to_e4m3fn(rng.normal(scale=40, size=(e, d, inter)).astype(np.float32))
    s2 = rng.uniform(2**-9, 2**-7, size=(e, d // 128, inter // 128)).astype(np.float32)
    return w1, s1, w2, s2


def test_expert_mlp_gate_then_up():
    rng = _rng(5)
    w1, s1, w2, s2 = _weights(rng, 1, 128, 128)
    x = rng.normal(size=(3, 128)).astype(np.float32)
    gu = moe.fp8_linear(x, w1[0], s1[0])
    h = gu[:, :128] / (1 + np.exp(-gu[:, :128].astype(np.float64))) * gu[:, 128:]
    want = moe.fp8_linear(h.astype(np.float32), w2[0], s2[0])
    np.testing.assert_allclose(moe.expert_mlp(x, w1[0], s1[0], w2[0], s2[0]), want, rtol=1e-4, atol=1e-3)
    swapped = moe.fp8_linear(
        (gu[:, 128:] / (1 + np.exp(-gu[:, 128:].astype(np.float64))) * gu[:, :128]).astype(np.float32), w2[0], s2[0])
    assert not np.allclose(swapped, want, rtol=1e-2)


def test_experts_combine_and_shared_slot():
    rng = _rng(6)
    e, inter, d, t = 3, 128, 128, 6
    w1, s1, w2, s2 = _weights(rng, e, inter, d)
    x = rng.normal(size=(t, d)).astype(np.float32)
    ids = np.array([[0], [1], [0], [1], [0], [1]], dtype=np.int32)
    w = rng.uniform(0.5, 1.5, size=(t, 1)).astype(np.float32)
    ids2, w2s = moe.with_shared_slot(ids, w, 2)
    assert ids2.shape == (t, 2) and np.all(ids2[:, 1] == 2) and np.all(w2s[:, 1] == 1.0)
    got = moe.moe_experts(x, ids2, w2s, w1, s1, w2, s2)
    for i in range(t):
        y_r = moe.expert_mlp(x[i:i + 1], w1[ids[i, 0]], s1[ids[i, 0]], w2[ids[i, 0]], s2[ids[i, 0]])
        y_s = moe.expert_mlp(x[i:i + 1], w1[2], s1[2], w2[2], s2[2])
        np.testing.assert_allclose(got[i], (w[i, 0] * y_r + y_s)[0], rtol=2e-4, atol=2e-3)


def test_sqnr_db():
    ref = np.ones(100)
    assert moe.sqnr_db(ref, ref) == float("inf")
    assert abs(moe.sqnr_db(ref, ref * 1.01) - 40.0) < 1e-6


def test_router_logits_round_the_fp32_product_to_bf16():
    # deepseek_v2/reference.py:173: rounded_to_bfloat16(x @ router_weight^T), the product in fp32.
    # Rows 0-2 are products exact in fp32 that sit on bf16 ties (ties to the even mantissa: 1 + 2**-8 ->
    # 1.0, 1 + 3 * 2**-8 -> 1 + 2**-6; a truncation, a round-half-up or a skipped rounding fails one).
    # Row 3's exact value 1 + 2**-8 + 2**-30 rounds to 1 + 2**-8 in fp32 in any summation order, then to
    # 1.0 in bf16; rounding the float64 product to bf16 directly would give 1 + 2**-7.
    x = np.array([[1.0, 2**-8, 0.0], [1.0, 3 * 2**-8, 0.0], [-1.0, -(2**-8), 0.0], [1.0, 2**-8, 2**-30]],
                 dtype=np.float32)
    w = np.array([[1.0, 1.0, 1.0], [2.0, 0.0, 0.0]], dtype=np.float32)
    got = moe.router_logits(x, w)
    want = np.array([[1.0, 2.0], [1.0 + 2**-6, 2.0], [-1.0, -2.0], [1.0, 2.0]], dtype=np.float32)
    assert got.dtype == np.float32 and np.array_equal(got, want)
    # orientation: logits[t, e] = sum_d x[t, d] * router_weight[e, d] (hand-computed, all exact)
    x = np.array([[1, 2, 3, 4], [0.5, 0, -1, 2]], dtype=np.float32)
    w = np.array([[1, 0, 0, 0], [0, 1, 1, 0], [0.25, 0.25, 0.25, 0.25]], dtype=np.float32)
    assert np.array_equal(moe.router_logits(x, w), np.array([[1, 5, 2.5], [0.5, -1, 0.375]], np.float32))


def test_composed_moe_on_forced_routing_equals_the_experts():
    # A router whose logits are known exactly (only column 0 of the router weight is non-zero and every
    # token has x[:, 0] = 1, so logits[t, e] = c[e]) and a bias of +1 on four chosen experts, two in each
    # of groups 0 and 1: those two groups are kept and the four are the picks, whatever the other scores.
    # The weights are then sigmoid(c) of the picks (unbiased), renormalized, times 2.5 -- computed here
    # in float64 -- and the shared expert adds at weight 1. A biased weight, a dropped scale factor or a
    # wrong shared-slot weight fails (the group axis is pinned by the per-token loop below).
    rng = _rng(7)
    n_routed, g, tg, topk, d, inter, t = 16, 4, 2, 4, 128, 128, 5
    w1, s1, w2, s2 = _weights(rng, n_routed + 1, inter, d)
    c = formats.round_to_bf16(rng.uniform(-2, 2, size=n_routed).astype(np.float32))
    wr = np.zeros((n_routed, d), np.float32)
    wr[:, 0] = c
    x = formats.round_to_bf16(rng.normal(size=(t, d)).astype(np.float32))
    x[:, 0] = 1.0
    chosen = [1, 2, 5, 6]
    bias = np.zeros(n_routed, np.float32)
    bias[chosen] = 1.0
    got = moe.deepseek_v2_fp8_moe(x, wr, bias, w1, s1, w2, s2, topk, g, tg, True, 2.5)
    sig = 1.0 / (1.0 + np.exp(-c.astype(np.float64)))
    order = sorted(chosen, key=lambda e: (-sig[e], e))
    wts = sig[order] / sig[order].sum() * 2.5
    ids = np.tile(np.array(order + [n_routed], np.int32), (t, 1))
    weights = np.tile(np.append(wts, 1.0).astype(np.float32), (t, 1))
    want = moe.moe_experts(x, ids, weights, w1, s1, w2, s2)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())
    # and the picks themselves
    r_ids, r_w = moe.grouped_topk(moe.router_logits(x, wr), bias, topk, g, tg, True, 2.5)
    assert np.array_equal(r_ids, ids[:, :topk])
    np.testing.assert_allclose(r_w, weights[:, :topk], rtol=1e-6)


def _brute_route(logit_row, bias, topk, n_groups, topk_group, factor):
    """One token's grouped top-k by explicit loops in float64 (deepseek_v2/reference.py:121-143): the
    group score as the two best biased scores summed, groups then experts taken by repeated maximum,
    the lower index first among equals."""
    import math

    scores = [1.0 / (1.0 + math.exp(-float(v))) for v in logit_row]
    biased = [s + float(b) for s, b in zip(scores, bias)]
    per = len(biased) // n_groups
    gscore = []
    for gi in range(n_groups):
        vals = sorted(biased[gi * per:(gi + 1) * per], reverse=True)
        gscore.append(vals[0] + vals[1])
    kept = []
    for _ in range(topk_group):
        kept.append(max((v, -i) for i, v in enumerate(gscore) if i not in kept)[1] * -1)
    ids = []
    for _ in range(topk):
        ids.append(max((biased[i], -i) for i in range(len(biased)) if i // per in kept and i not in ids)[1] * -1)
    w = [scores[i] for i in ids]
    return ids, [v / sum(w) * factor for v in w]


def test_composed_moe_against_a_per_token_loop():
    # the whole oracle op against an independent per-token construction: logits by exact sums (fsum)
    # rounded to fp32 then bf16, the routing by _brute_route, each token's slots through the pinned
    # expert MLP one token at a time, the shared expert last at weight 1
    import math

    rng = _rng(8)
    n_routed, g, tg, topk, d, inter, t = 16, 4, 2, 4, 128, 128, 6
    w1, s1, w2, s2 = _weights(rng, n_routed + 1, inter, d)
    x = formats.round_to_bf16(rng.normal(size=(t, d)).astype(np.float32))
    wr = formats.round_to_bf16(rng.normal(scale=0.2, size=(n_routed, d)).astype(np.float32))
    bias = formats.round_to_bf16(rng.normal(scale=0.05, size=n_routed).astype(np.float32))
    got = moe.deepseek_v2_fp8_moe(x, wr, bias, w1, s1, w2, s2, topk, g, tg, True, 2.5)
    for i in range(t):
        logit = [formats.round_to_bf16(np.array([math.fsum(float(a) * float(b) for a, b in zip(x[i], wr[e]))],
                                                np.float32))[0] for e in range(n_routed)]
        ids, wts = _brute_route(logit, bias, topk, g, tg, 2.5)
        want = moe.expert_mlp(x[i:i + 1], w1[n_routed], s1[n_routed], w2[n_routed], s2[n_routed])[0].astype(np.float64)
        for e, wt in zip(ids, wts):
            want += wt * moe.expert_mlp(x[i:i + 1], w1[e], s1[e], w2[e], s2[e])[0]
        np.testing.assert_allclose(got[i], want, rtol=2e-4, atol=2e-4 * np.abs(want).max())

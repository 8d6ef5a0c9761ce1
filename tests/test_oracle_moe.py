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

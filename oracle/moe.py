"""Grouped DeepSeek FP8 MoE (deepseek_v2_fp8_moe), restated in numpy (test infrastructure; see
``oracle/__init__.py``).

Follows aklr/plugins/sglang/models/deepseek_v2/reference.py:
- router logits: fp32 ``x @ router_weight^T`` rounded to bf16 (:173);
- ``_grouped_routed`` (:121-143): scores = sigmoid(logits); biased = scores + correction_bias;
  experts fall into num_expert_group equal groups, a group scored by its two best biased scores
  summed; the topk_group best groups are kept (lower index first among equals, ``_first_largest``
  :111-118); each token's topk experts are its best biased scores among the kept groups' experts
  (lower index first among equals); weights are the UNBIASED scores of those experts, divided by
  their sum when renormalize, times routed_scaling_factor;
- ``_with_shared_slot`` (:80-89): the shared expert (index n_routed) appended as a last slot at weight 1;
- ``_fp8_linear`` (:146-160): the input rounded to bf16, each 1 x 128 group scaled by
  ``amax / 448`` -- a true division (unlike per_group_quant_fp8's multiply by fl32(1/448)) --
  clamped below at the fp32 tiny (2**-126), cast to e4m3fn (round to nearest even), dequantized,
  then multiplied by the block-dequantized weight [n, k] (scale per 128 x 128 block);
- ``_experts`` / ``_mlp`` (:41-46, :64-77, :178-181): per expert, gate and up are the two halves of
  the first linear's output, ``silu(gate) * up`` feeds the second linear, and each token's rows are
  weighed and summed.

Arithmetic: fp32 everywhere the reference is fp32; the matrix products accumulate in float64 and
round to fp32 (the reference's fp32 matmul differs from that only at the ulp level, which the
contract's SQNR >= 30 dB bound does not see).

Pinned in tests/test_oracle_moe.py by: ungrouped routing reducing to a plain top-k of the biased
scores (checked against an independent argpartition), the kept-group invariants on grouped routing,
explicit ties (lower index first), weights from the unbiased scores (a bias that changes the picks
but not the weights), the division-vs-multiply scale on values where the two differ in fp32,
``_fp8_linear`` reducing to the pinned a8w8 GEMM oracle, and the combine on one-expert and
shared-only routings. ``router_logits`` by products exact in fp32 that sit on bf16 ties (ties to even)
and one whose fp32 rounding decides the bf16 value (so the product is rounded to fp32 first, as the
reference's fp32 matmul is); the composed ``deepseek_v2_fp8_moe`` by reduction to ``moe_experts`` on a
forced routing with hand-computed weights, and against a per-token loop that routes by repeated
maximum in float64.
"""
from __future__ import annotations

import numpy as np

from .formats import f32_to_e4m3fn, round_to_bf16
from .gemm import dequant_b8, dequant_a8

FP32_TINY = np.float32(np.finfo(np.float32).tiny)
FP8_MAX = np.float32(448.0)


def sigmoid32(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    return (np.float32(1.0) / (np.float32(1.0) + np.exp(-x).astype(np.float32))).astype(np.float32)


def router_logits(x: np.ndarray, router_weight: np.ndarray) -> np.ndarray:
    """x float32 [T, D], router_weight float32 [E, D] -> bf16-valued float32 logits [T, E]."""
    prod = (x.astype(np.float64) @ router_weight.astype(np.float64).T).astype(np.float32)
    return round_to_bf16(prod)


def _first_largest(values: np.ndarray, k: int) -> np.ndarray:
    """Indices of each row's k largest values, the lower index first among equals."""
    return np.argsort(-values, axis=-1, kind="stable")[..., :k]


def grouped_topk(logits: np.ndarray, bias: np.ndarray, topk: int, num_expert_group: int, topk_group: int,
                 renormalize: bool, routed_scaling_factor: float) -> tuple[np.ndarray, np.ndarray]:
    """logits float32 [T, E] (bf16 values), bias float32 [E] -> (ids int32 [T, topk], weights
    float32 [T, topk]), ids in descending order of biased score."""
    scores = sigmoid32(logits)
    biased = (scores + np.asarray(bias, dtype=np.float32)).astype(np.float32)
    t, e = biased.shape
    per = e // num_expert_group
    groups = biased.reshape(t, num_expert_group, per)
    top2 = -np.sort(-groups, axis=-1)[..., :2]
    group_scores = (top2[..., 0] + top2[..., 1]).astype(np.float32)
    kept = np.zeros((t, num_expert_group), dtype=bool)
    np.put_along_axis(kept, _first_largest(group_scores, topk_group), True, axis=-1)
    allowed = np.repeat(kept, per, axis=-1)
    masked = np.where(allowed, biased, np.float32(-np.inf))
    ids = _first_largest(masked, topk)
    weights = np.take_along_axis(scores, ids, axis=-1).astype(np.float32)
    if renormalize:
        weights = (weights / weights.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    weights = (weights * np.float32(routed_scaling_factor)).astype(np.float32)
    return ids.astype(np.int32), weights


def with_shared_slot(ids: np.ndarray, weights: np.ndarray, n_routed: int) -> tuple[np.ndarray, np.ndarray]:
    t = ids.shape[0]
    ids = np.concatenate([ids, np.full((t, 1), n_routed, dtype=np.int32)], axis=-1)
    weights = np.concatenate([weights, np.ones((t, 1), dtype=np.float32)], axis=-1)
    return ids, weights


def quant_fp8_div(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The fp8 linear's input quantization: float32 [R, K] -> (e4m3fn codes [R, K], scales
    float32 [R, K/128]); input rounded to bf16, scale = max(amax / 448, tiny), codes = e4m3(x / s)."""
    xb = round_to_bf16(np.asarray(x, dtype=np.float32))
    r, k = xb.shape
    g = xb.reshape(r, k // 128, 128)
    amax = np.abs(g).max(axis=-1).astype(np.float32)
    scale = np.maximum((amax / FP8_MAX).astype(np.float32), FP32_TINY)
    q = f32_to_e4m3fn((g / scale[..., None]).astype(np.float32)).reshape(r, k)
    return q, scale


def fp8_linear(x: np.ndarray, w_codes: np.ndarray, w_scale: np.ndarray) -> np.ndarray:
    """x float32 [R, K]; w e4m3fn codes [N, K], w_scale float32 [ceil(N/128), K/128] -> [R, N]."""
    q, s = quant_fp8_div(x)
    xd = dequant_a8(q, s)
    wd = dequant_b8(w_codes, w_scale)
    return (xd.astype(np.float64) @ wd.astype(np.float64).T).astype(np.float32)


def silu32(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    return (x * sigmoid32(x)).astype(np.float32)


def expert_mlp(rows: np.ndarray, w1: np.ndarray, s1: np.ndarray, w2: np.ndarray, s2: np.ndarray) -> np.ndarray:
    """rows float32 [R, D]; w1 [2I, D] (gate rows, then up rows), w2 [D, I] -> [R, D]."""
    gu = fp8_linear(rows, w1, s1)
    inter = gu.shape[1] // 2
    h = (silu32(gu[:, :inter]) * gu[:, inter:]).astype(np.float32)
    return fp8_linear(h, w2, s2)


def moe_experts(x: np.ndarray, ids: np.ndarray, weights: np.ndarray, w1: np.ndarray, s1: np.ndarray,
                w2: np.ndarray, s2: np.ndarray) -> np.ndarray:
    """x float32 [T, D]; ids/weights [T, S] (every slot, shared included); w1 [E, 2I, D], s1
    [E, 2I/128, D/128], w2 [E, D, I], s2 [E, D/128, I/128] -> float32 [T, D]."""
    out = np.zeros(x.shape, dtype=np.float32)
    for e in np.unique(ids).tolist():
        tokens, slots = np.nonzero(ids == e)
        y = expert_mlp(x[tokens], w1[e], s1[e], w2[e], s2[e])
        np.add.at(out, tokens, (weights[tokens, slots][:, None] * y).astype(np.float32))
    return out


def deepseek_v2_fp8_moe(x: np.ndarray, router_weight: np.ndarray, correction_bias: np.ndarray, w1: np.ndarray,
                        s1: np.ndarray, w2: np.ndarray, s2: np.ndarray, topk: int, num_expert_group: int,
                        topk_group: int, renormalize: bool, routed_scaling_factor: float) -> np.ndarray:
    """The whole op on float32 inputs (bf16 values); the routed experts then the shared one (the
    last of w1/w2's n_routed + 1 slots). Returns float32 [T, D] (the op's output before its bf16
    rounding)."""
    n_routed = router_weight.shape[0]
    logits = router_logits(x, router_weight)
    ids, weights = grouped_topk(logits, correction_bias, topk, num_expert_group, topk_group, renormalize,
                                routed_scaling_factor)
    ids, weights = with_shared_slot(ids, weights, n_routed)
    return moe_experts(x, ids, weights, w1, s1, w2, s2)


def sqnr_db(ref: np.ndarray, got: np.ndarray) -> float:
    """20 log10(||ref|| / ||got - ref||), the contract's SqnrBound
    (aklr/core/contract/semantics/_compare.py:424-466); callers pass the reference already rounded
    to the output dtype, as that bound does."""
    ref = np.asarray(ref, dtype=np.float64)
    err = np.asarray(got, dtype=np.float64) - ref
    num, den = float((ref * ref).sum()), float((err * err).sum())
    if den == 0.0:
        return float("inf")
    return 10.0 * np.log10(num / den) if num > 0 else float("-inf")

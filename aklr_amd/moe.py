"""Grouped DeepSeek FP8 MoE: the reference's op signature over the HIP kernels.

``deepseek_v2_fp8_moe`` -- aklr/plugins/sglang/models/deepseek_v2/api.py:35-50, contract
deepseek_v2/contract.py:188-320 (``deepseek_v2_fp8_moe@1.0``), arithmetic deepseek_v2/reference.py:146-183:
sglang's DeepseekV2MoE on one rank. Router logits in bf16, sigmoid scores, grouped top-k on the scores
plus correction_bias (groups scored by their two best), weights = renormalized unbiased scores times
routed_scaling_factor, the shared expert (the last of w1/w2's slots) at weight 1; each expert
down(silu(gate(x)) * up(x)) with 128x128-block-scaled fp8 linears whose inputs are quantized per 1x128
at scale amax / 448.
  In contract (contract.py:222-260, the attrs' listed values): topk 8; (num_expert_group, topk_group)
  (8, 4) or (1, 1); renormalize True; scoring_func "sigmoid"; routed_scaling_factor 2.5; hidden and
  router_weight bf16, correction_bias bf16, w1/w2 e4m3fn, scales fp32; the axis domains and
  constraints of :211-240. Anything else returns OUT_OF_CONTRACT, never raises.
  Variants (contract.py:307-318): ``row_major`` (w1 and w2 not marked ``is_shuffled``) and
  ``shuffled_16x16`` (both marked: aiter shuffle_weight per expert).

``moe_fp8_route`` and ``moe_fp8_experts`` are the op's two halves on their own, with the general
arguments the kernels take (any topk <= 63, group counts, scale factor, slot count): the grouped top-k
of reference.py:121-143 (+ the shared slot, :80-89), and the experts on a given routing -- the role of
aiter fused_moe(per_128x128) in the reference's baseline (deepseek_v2/baseline.py:152-163). They raise
``ValueError`` on arguments the kernels cannot take.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import _lib
from .dispatch import FallbackReason, aligned, api, on_gpu

CONTRACT_ID = "deepseek_v2_fp8_moe@1.0"
_OOC = FallbackReason.OUT_OF_CONTRACT
_FP8 = torch.float8_e4m3fn


def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _w_layout(w1, w2):
    """The weights' layout, or None when the two disagree (no variant matches)."""
    s1 = getattr(w1, "is_shuffled", False) is True
    s2 = getattr(w2, "is_shuffled", False) is True
    if s1 != s2:
        return None
    return ("shuffled_16x16", _lib.B_PRESHUFFLE_16x16) if s1 else ("row_major", _lib.B_ROW_MAJOR)


def _weights_ok(w1, w1_scale, w2, w2_scale, experts, d, inter) -> bool:
    if w1.dtype != _FP8 or w2.dtype != _FP8 or w1_scale.dtype != torch.float32 or w2_scale.dtype != torch.float32:
        return False
    if tuple(w1.shape) != (experts, 2 * inter, d) or tuple(w2.shape) != (experts, d, inter):
        return False
    if tuple(w1_scale.shape) != (experts, 2 * inter // 128, d // 128):
        return False
    if tuple(w2_scale.shape) != (experts, d // 128, inter // 128):
        return False
    return all(t.is_contiguous() for t in (w1, w1_scale, w2, w2_scale))


@dataclass
class _MoePlan:
    hidden: torch.Tensor
    router_weight: torch.Tensor
    correction_bias: torch.Tensor
    w1: torch.Tensor
    w1_scale: torch.Tensor
    w2: torch.Tensor
    w2_scale: torch.Tensor
    tokens: int
    d: int
    inter: int
    n_routed: int
    topk: int
    groups: int
    topk_group: int
    scale: float
    w_layout: int
    variant: str
    kernel_ref: str = field(default="aklr_deepseek_v2_fp8_moe:grouped")


_I32_LIMIT = 0x7FFFFFFE  # the kernels' 32-bit byte offsets stay below 2 GiB


def token_chunks(tokens: int, d: int, inter: int, slots: int) -> list[tuple[int, int]]:
    """[start, end) token ranges one library call each can take. The kernels address the routed rows'
    activations (R x D bf16), the intermediate h (R x I) and the input (T x D) with 32-bit offsets,
    R = tokens x slots, so the library takes at most that many tokens per call (the limits of its
    dims_ok); every token's output depends on that token alone (its routing, its rows through the
    experts, its combine), so a larger call runs as consecutive calls on row ranges."""
    most = min(65536, _I32_LIMIT // (2 * d * slots), _I32_LIMIT // (inter * slots), _I32_LIMIT // d)
    if most < 1:
        return []
    return [(s, min(tokens, s + most)) for s in range(0, tokens, most)]


def _run_moe(p: _MoePlan):
    dev = p.hidden.device
    out = torch.empty((p.tokens, p.d), dtype=torch.bfloat16, device=dev)
    L = _lib.lib()
    chunks = token_chunks(p.tokens, p.d, p.inter, p.topk + 1)
    most = max(e - s for s, e in chunks)
    ws_bytes = L.aklr_moe_fp8_workspace_bytes(most, p.d, p.inter, p.n_routed + 1, p.topk + 1, p.n_routed)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    row = p.d * 2  # bytes per hidden / out row
    for s, e in chunks:
        st = L.aklr_deepseek_v2_fp8_moe(
            p.hidden.data_ptr() + s * row, p.router_weight.data_ptr(), p.correction_bias.data_ptr(), p.w1.data_ptr(),
            p.w1_scale.data_ptr(), p.w2.data_ptr(), p.w2_scale.data_ptr(), e - s, p.d, p.inter, p.n_routed, p.topk,
            p.groups, p.topk_group, 1, p.scale, p.w_layout, out.data_ptr() + s * row, ws.data_ptr(), ws_bytes,
            _stream(dev),
        )
        _lib.check(st, "deepseek_v2_fp8_moe")
    return out


@api(CONTRACT_ID, _run_moe)
def deepseek_v2_fp8_moe(
    hidden_states,
    router_weight,
    correction_bias,
    w1,
    w1_scale,
    w2,
    w2_scale,
    topk,
    num_expert_group,
    topk_group,
    renormalize,
    scoring_func,
    routed_scaling_factor,
):
    tensors = (hidden_states, router_weight, correction_bias, w1, w1_scale, w2, w2_scale)
    if not all(isinstance(t, torch.Tensor) for t in tensors):
        return _OOC
    # attrs and scalar at the contract's listed values (contract.py:222-240, :290-296)
    if topk != 8 or (num_expert_group, topk_group) not in ((8, 4), (1, 1)) or renormalize is not True:
        return _OOC
    if scoring_func != "sigmoid" or routed_scaling_factor != 2.5:
        return _OOC
    # dtypes
    if hidden_states.dtype != torch.bfloat16 or router_weight.dtype != hidden_states.dtype:
        return _OOC
    if correction_bias.dtype != torch.bfloat16:
        return _OOC
    # shapes and axis domains (contract.py:211-221) and constraints (:241-248)
    if hidden_states.dim() != 2 or router_weight.dim() != 2 or correction_bias.dim() != 1:
        return _OOC
    tokens, d = hidden_states.shape
    n_routed = router_weight.shape[0]
    if w1.dim() != 3 or w2.dim() != 3:
        return _OOC
    inter = w2.shape[2]
    if not (1 <= tokens <= 65536 and 128 <= d <= 16384 and d % 128 == 0 and 1 <= n_routed <= 1024):
        return _OOC
    if not (128 <= inter <= 16384 and inter % 128 == 0):
        return _OOC
    if router_weight.shape[1] != d or tuple(correction_bias.shape) != (n_routed,):
        return _OOC
    if n_routed % num_expert_group or n_routed // num_expert_group < 2 or topk > topk_group * (n_routed // num_expert_group):
        return _OOC
    if not _weights_ok(w1, w1_scale, w2, w2_scale, n_routed + 1, d, inter):
        return _OOC
    if not all(t.is_contiguous() for t in (hidden_states, router_weight, correction_bias)):
        return _OOC
    layout = _w_layout(w1, w2)
    if layout is None:
        return _OOC
    if not on_gpu(*tensors) or not all(aligned(t) for t in tensors):
        return _OOC
    variant, w_layout = layout
    return _MoePlan(hidden_states, router_weight, correction_bias, w1, w1_scale, w2, w2_scale, tokens, d, inter,
                    n_routed, topk, num_expert_group, topk_group, float(routed_scaling_factor), w_layout, variant)


# ---------------------------------------------------------------------------------------------
def moe_fp8_route(logits, correction_bias, topk, num_expert_group=1, topk_group=1, renormalize=True,
                  routed_scaling_factor=1.0, append_shared=True):
    """Grouped top-k on bf16 logits [T, E] -> (ids int32 [T, S], weights fp32 [T, S]), S = topk (+1 with
    the shared slot, expert E at weight 1). Ids in descending biased score, lower index first on ties."""
    if logits.dtype != torch.bfloat16 or correction_bias.dtype != torch.bfloat16:
        raise ValueError("moe_fp8_route takes bf16 logits and a bf16 correction_bias")
    if not (logits.is_cuda and correction_bias.device == logits.device):
        raise ValueError("moe_fp8_route runs on one GPU")
    logits = logits.contiguous()
    correction_bias = correction_bias.contiguous()
    t, e = logits.shape
    slots = topk + (1 if append_shared else 0)
    ids = torch.empty((t, slots), dtype=torch.int32, device=logits.device)
    weights = torch.empty((t, slots), dtype=torch.float32, device=logits.device)
    st = _lib.lib().aklr_moe_fp8_route(
        logits.data_ptr(), correction_bias.data_ptr(), t, e, topk, num_expert_group, topk_group, int(bool(renormalize)),
        float(routed_scaling_factor), int(bool(append_shared)), ids.data_ptr(), weights.data_ptr(),
        _stream(logits.device),
    )
    if st == _lib.AKLR_ERR_INVALID_ARGUMENT:
        raise ValueError("moe_fp8_route: arguments outside what the kernel takes")
    _lib.check(st, "moe_fp8_route")
    return ids, weights


def moe_fp8_experts(hidden_states, w1, w2, topk_weights, topk_ids, w1_scale, w2_scale):
    """out[t] = sum over slots s of topk_weights[t, s] * expert_{topk_ids[t, s]}(hidden_states[t]), each
    expert down(silu(gate) * up) of 128x128-block-scaled fp8 weights (w1 [E, 2I, D], w2 [E, D, I], per
    expert row-major or, when both carry ``is_shuffled``, aiter-preshuffled); ids outside [0, E) are
    skipped. Returns bf16 [T, D]."""
    layout = _w_layout(w1, w2)
    if layout is None:
        raise ValueError("w1 and w2 must share one layout")
    if hidden_states.dtype != torch.bfloat16:
        raise ValueError("hidden_states must be bf16")
    if not on_gpu(hidden_states, w1, w2, topk_weights, topk_ids, w1_scale, w2_scale):
        raise ValueError("moe_fp8_experts runs on one GPU")
    t, d = hidden_states.shape
    e, inter = w1.shape[0], w2.shape[2]
    if not _weights_ok(w1, w1_scale, w2, w2_scale, e, d, inter):
        raise ValueError("expert weights / scales do not have the [E, 2I, D] / [E, D, I] fp8 layout")
    hidden_states = hidden_states.contiguous()
    ids = topk_ids.to(torch.int32).contiguous()
    weights = topk_weights.to(torch.float32).contiguous()
    if ids.shape != weights.shape or ids.dim() != 2 or ids.shape[0] != t:
        raise ValueError("topk_ids and topk_weights must both be [T, slots]")
    slots = ids.shape[1]
    L = _lib.lib()
    chunks = token_chunks(t, d, inter, slots)
    ws_bytes = L.aklr_moe_fp8_workspace_bytes(max((b - a for a, b in chunks), default=0), d, inter, e, slots, 0)
    if ws_bytes == 0:
        raise ValueError("moe_fp8_experts: sizes outside what the kernels take")
    out = torch.empty((t, d), dtype=torch.bfloat16, device=hidden_states.device)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=hidden_states.device)
    for a, b in chunks:
        st = L.aklr_moe_fp8_experts(
            hidden_states.data_ptr() + a * d * 2, b - a, d, inter, e, ids.data_ptr() + a * slots * 4,
            weights.data_ptr() + a * slots * 4, slots, w1.data_ptr(), w1_scale.data_ptr(), w2.data_ptr(),
            w2_scale.data_ptr(), layout[1], out.data_ptr() + a * d * 2, ws.data_ptr(), ws_bytes,
            _stream(hidden_states.device),
        )
        _lib.check(st, "moe_fp8_experts")
    return out

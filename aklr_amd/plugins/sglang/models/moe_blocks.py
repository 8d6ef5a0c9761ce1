# SPDX-License-Identifier: MIT
# Copyright (C) 2025-2026, Advanced Micro Devices, Inc. All rights reserved.
# The host protocol and rules here follow aklr/plugins/sglang/models/moe_blocks.py, whose licence notice this is.

"""The checks that keep a sglang MoE call on sglang (aklr/plugins/sglang/models/moe_blocks.py:16-126).

They read sglang's own state: the graph mode and parallel configuration of the running model, and how
a FusedMoE layer holds its experts. The op itself declines shapes and dtypes; these checks cover what
the op cannot see from its arguments: expert parallelism, redundant or relocated experts, recorders,
and experts that sglang runs in another format or with another activation than the op's.
"""
from __future__ import annotations

__all__ = ["experts_fall_back", "experts_format", "runtime_falls_back"]


def runtime_falls_back() -> bool:
    """Whether sglang's graph mode or parallel/expert configuration keeps MoE calls on sglang."""
    from sglang.srt.environ import envs
    from sglang.srt.layers.moe import get_moe_a2a_backend
    from sglang.srt.model_executor.runner_backend_utils.breakable_cuda_graph.context import (
        is_in_breakable_cuda_graph,
    )
    from sglang.srt.model_executor.runner_backend_utils.tc_piecewise_cuda_graph.context_manager import (
        is_in_tc_piecewise_cuda_graph,
    )
    from sglang.srt.runtime_context import get_exec, get_parallel

    exe, parallel = get_exec(), get_parallel()
    moe = exe.moe
    if is_in_tc_piecewise_cuda_graph() or is_in_breakable_cuda_graph():
        return True  # captured piecewise: sglang owns the call
    if not get_moe_a2a_backend().is_none() or moe.ep_join_mode is not None or parallel.dwdp_size > 1:
        return True  # tokens travel between ranks: the op runs one rank's whole expert set
    if moe.enable_eplb or moe.enable_waterfill or moe.init_expert_location != "trivial":
        return True  # experts relocated or rebalanced
    if moe.ep_num_redundant_experts > 0 or moe.expert_distribution_recorder_mode is not None:
        return True
    if exe.deterministic.enable_deterministic_inference or exe.features.enable_return_routed_experts:
        return True
    return bool(envs.SGLANG_SIMULATE_UNIFORM_EXPERTS.get() or envs.SGLANG_SIMULATE_ROUND_ROBIN_EXPERTS.get())


def experts_format(experts) -> str:
    """The name of the class that defines how ``experts`` are stored: their scheme's, else their
    quantization method's (sglang's own rule)."""
    return type(getattr(experts, "scheme", None) or experts.quant_method).__name__


def experts_fall_back(experts, formats: tuple[str, ...]) -> bool:
    """Whether ``experts`` run other than the op takes them: a format outside ``formats``, not a plain
    FusedMoE at sglang's standard dispatch, or not gated silu on aiter's fused_moe."""
    if experts_format(experts) not in formats:
        return True
    if type(experts).__name__ != "FusedMoE" or type(experts.dispatcher).__name__ != "StandardDispatcher":
        return True
    if experts.reduce_results:
        return True
    runner = _fp8_block_runner(experts)
    if runner is None or not runner.runner_backend.is_aiter():
        return True
    config = runner.config
    if config.activation != "silu" or not config.is_gated:
        return True
    if config.apply_router_weight_on_input or config.no_combine:
        return True
    if config.gemm1_alpha is not None or config.gemm1_clamp_limit is not None:
        return True
    if config.swiglu_limit not in (None, 0.0):  # aiter clamps only at a limit other than 0
        return True
    if getattr(experts, "w13_weight_bias", None) is not None or getattr(experts, "w2_weight_bias", None) is not None:
        return True
    return bool(getattr(experts, "fp8_activations", False))


def _fp8_block_runner(experts):
    """The runner of fp8 experts with one scale per 128 x 128 block -- the op's format -- else None."""
    if experts_format(experts) != "Fp8MoEMethod":
        return None
    method = experts.quant_method
    if not method.block_quant or method.use_mxfp8 or method.is_fp4_expert:
        return None
    if list(method.weight_block_size) != [128, 128]:
        return None
    return getattr(method, "runner", None)

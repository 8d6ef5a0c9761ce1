"""aklr_amd -- MI355X (gfx950) block-scaled FP8 / MXFP4 GEMM path, drop-in for AKLR's.

Ops keep the reference's signatures (aklr/ops/quant/api.py, aklr/ops/gemm/api.py,
aklr/plugins/sglang/models/deepseek_v2/api.py) and return their
outputs or a ``FallbackReason``. They run hand-written HIP kernels through the C ABI of
``include/aklr_amd.h`` (``libaklr_amd.so``, built in-tree by ``aklr_amd._build``).
"""
from .dispatch import FallbackReason, KernelInfo
from .gemm import gemm_a4w4_mxfp4, gemm_a8w8_blockwise_scaled, quant_gemm_a8w8_blockwise_scaled
from .moe import deepseek_v2_fp8_moe, moe_fp8_experts, moe_fp8_route
from .quant import dynamic_mxfp4_quant, per_group_quant_fp8, per_group_quant_mxfp8

__all__ = [
    "FallbackReason",
    "KernelInfo",
    "deepseek_v2_fp8_moe",
    "dynamic_mxfp4_quant",
    "gemm_a4w4_mxfp4",
    "gemm_a8w8_blockwise_scaled",
    "moe_fp8_experts",
    "moe_fp8_route",
    "per_group_quant_fp8",
    "per_group_quant_mxfp8",
    "quant_gemm_a8w8_blockwise_scaled",
]

"""aklr_amd -- MI355X (gfx950) block-scaled FP8 / MXFP4 GEMM path, drop-in for AKLR's.

Ops keep the reference's signatures (aklr/ops/quant/api.py, aklr/ops/gemm/api.py) and return their
outputs or a ``FallbackReason``. They run hand-written HIP kernels through the C ABI of
``include/aklr_amd.h`` (``libaklr_amd.so``, built in-tree by ``aklr_amd._build``).
"""
from .dispatch import FallbackReason, KernelInfo
from .gemm import gemm_a4w4_mxfp4, gemm_a8w8_blockwise_scaled
from .quant import dynamic_mxfp4_quant, per_group_quant_fp8, per_group_quant_mxfp8

__all__ = [
    "FallbackReason",
    "KernelInfo",
    "dynamic_mxfp4_quant",
    "gemm_a4w4_mxfp4",
    "gemm_a8w8_blockwise_scaled",
    "per_group_quant_fp8",
    "per_group_quant_mxfp8",
]

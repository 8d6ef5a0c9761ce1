"""Activation quantization ops: the reference's op signatures over the HIP kernels.

- ``per_group_quant_fp8(x)`` -- aklr/ops/quant/api.py:8-9, contract aklr/ops/quant/contract.py:17-51:
  bf16 [T, H] (H % 128 == 0) -> (e4m3fn [T, H], fp32 dequant scales [H/128, T] group-major).
- ``per_group_quant_mxfp8(x)`` -- aklr/ops/quant/api.py:12-13, contract :54-75:
  bf16 [T, H] (H % 32 == 0) -> (e4m3fn [T, H], uint8 e8m0 exponents [T, H/32]).
- ``dynamic_mxfp4_quant(x, shuffle=False)`` -- the MXFP4 activation quantizer the reference restates
  from aiter (aklr/ops/fused_moe/reference.py:21-37; no AKLR op exists): bf16 [T, H] (H % 32 == 0) ->
  (fp4x2 [T, H/2], e8m0 scales [T, H/32], or with ``shuffle`` the aiter padded/shuffled layout).

Each returns its outputs, or a ``FallbackReason`` for a call outside the contract (CPU tensors
included); the kernels run on the current stream of x's device.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .dispatch import FallbackReason, aligned, api, on_gpu

_MAX_TOKENS = 131072
_MAX_HIDDEN = 21504
# dynamic_mxfp4_quant feeds gemm_a4w4_mxfp4, whose K reaches 65536 (aklr/ops/gemm/contract.py:143)
_MAX_HIDDEN_MXFP4 = 65536
_E8M0 = getattr(torch, "float8_e8m0fnu", torch.uint8)
_FP4X2 = getattr(torch, "float4_e2m1fn_x2", torch.uint8)


def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _x_ok(x, multiple: int, max_hidden: int = _MAX_HIDDEN):
    if not isinstance(x, torch.Tensor) or x.dim() != 2 or x.dtype != torch.bfloat16:
        return False
    if not on_gpu(x) or not x.is_contiguous() or not aligned(x):
        return False
    t, h = x.shape
    return 1 <= t <= _MAX_TOKENS and multiple <= h <= max_hidden and h % multiple == 0


@dataclass
class _QuantPlan:
    x: torch.Tensor
    variant: str
    kernel_ref: str
    shuffle: bool = False


# ---------------------------------------------------------------------------------------------
def _run_fp8(p: _QuantPlan):
    x = p.x
    t, h = x.shape
    q = torch.empty((t, h), dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty((h // 128, t), dtype=torch.float32, device=x.device)
    st = _lib.lib().aklr_per_group_quant_fp8(x.data_ptr(), h, q.data_ptr(), s.data_ptr(), t, h, _stream(x.device))
    _lib.check(st, "per_group_quant_fp8")
    return q, s


@api("per_group_quant_fp8@1.0", _run_fp8)
def per_group_quant_fp8(x):
    if not _x_ok(x, 128):
        return FallbackReason.OUT_OF_CONTRACT
    return _QuantPlan(x, "row_major", "aklr_per_group_quant_fp8")


# ---------------------------------------------------------------------------------------------
def _run_mxfp8(p: _QuantPlan):
    x = p.x
    t, h = x.shape
    q = torch.empty((t, h), dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty((t, h // 32), dtype=torch.uint8, device=x.device)
    st = _lib.lib().aklr_per_group_quant_mxfp8(x.data_ptr(), h, q.data_ptr(), s.data_ptr(), t, h,
                                               _stream(x.device))
    _lib.check(st, "per_group_quant_mxfp8")
    return q, s


@api("per_group_quant_mxfp8@1.0", _run_mxfp8)
def per_group_quant_mxfp8(x):
    if not _x_ok(x, 32):
        return FallbackReason.OUT_OF_CONTRACT
    return _QuantPlan(x, "row_major", "aklr_per_group_quant_mxfp8")


# ---------------------------------------------------------------------------------------------
def mxfp4_scale_storage_shape(rows: int, groups: int, shuffle: bool) -> tuple[int, int]:
    """Storage shape of e8m0 scales: [rows, groups], or padded to (256, 8) multiples when shuffled
    (E8M0Scales(pad_to=(256, 8)), aklr/core/contract/semantics/_layouts.py:124-156)."""
    if not shuffle:
        return rows, groups
    return -(-rows // 256) * 256, -(-groups // 8) * 8


def _run_mxfp4(p: _QuantPlan):
    x = p.x
    t, h = x.shape
    q = torch.empty((t, h // 2), dtype=torch.uint8, device=x.device)
    s = torch.empty(mxfp4_scale_storage_shape(t, h // 32, p.shuffle), dtype=torch.uint8, device=x.device)
    layout = _lib.SCALES_SHUFFLED if p.shuffle else _lib.SCALES_ROW_MAJOR
    st = _lib.lib().aklr_dynamic_mxfp4_quant(x.data_ptr(), h, q.data_ptr(), s.data_ptr(), t, h, layout,
                                             _stream(x.device))
    _lib.check(st, "dynamic_mxfp4_quant")
    return q.view(_FP4X2), s.view(_E8M0)


@api("dynamic_mxfp4_quant@1.0", _run_mxfp4)
def dynamic_mxfp4_quant(x, shuffle=False):
    if not _x_ok(x, 32, _MAX_HIDDEN_MXFP4) or shuffle not in (True, False):
        return FallbackReason.OUT_OF_CONTRACT
    return _QuantPlan(x, "shuffled_scales" if shuffle else "row_major", "aklr_dynamic_mxfp4_quant", bool(shuffle))

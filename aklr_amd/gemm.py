"""Block-scaled GEMM ops: the reference's op signatures over the HIP kernels.

``gemm_a8w8_blockwise_scaled`` -- aklr/ops/gemm/api.py:32-46, contract aklr/ops/gemm/contract.py:211-308:
    out = (a * a_scale per 1x128) @ (b * b_scale per 128x128)^T + bias, fp32 accumulation, bf16/fp16 out.
  Layout variants (contract.py:280-307), detected exactly as the reference does:
    row_major                    operand_format "none:none", b not marked ``is_shuffled``;
    b_shuffled                   "none:preshuffled", a_scale not marked ``is_row_major``: b in aiter's
                                 16x16 shuffle_weight layout, a_scale column-major (the group-major
                                 bytes per_group_quant_fp8 writes; also accepted as a (1, m)-strided view);
    b_shuffled_row_major_a_scale "none:preshuffled", a_scale.is_row_major = True.
  Constraint (contract.py:242-246): the shuffled variants take trans_b, K-major scales, no bias, e4m3.
  trans_b = False (row_major; b is (k, n), contract.py:61-76): b is transposed on the GPU into (n, k)
  scratch (aklr_transpose_b8), then the same GEMM runs.
``gemm_a4w4_mxfp4`` -- aklr/ops/gemm/api.py:49-63, contract aklr/ops/gemm/contract.py:315-390:
    out = alpha * (a * 2^(a_scale-127)) @ (b * 2^(b_scale-127))^T + bias, alpha = 1, beta = 0, NT only.
  Variants: row_major ("none:none") and b_shuffled ("none:preshuffled", the default): preshuffled b and
  aiter's padded, shuffled e8m0 scales for both operands.

Calls the kernels do not serve return a ``FallbackReason`` (never raise): outside the contract ->
OUT_OF_CONTRACT (the in-contract rules of aklr/core/contract/fastkey/_fast_key_fn.py: dtypes, shapes,
strides, 16-byte alignment, one device, no output/input overlap).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import _lib, workspace
from .dispatch import FallbackReason, aligned, api, on_gpu, overlaps

_FP8 = {torch.float8_e4m3fn: _lib.FP8_E4M3FN, torch.float8_e5m2: _lib.FP8_E5M2}
_OUT = {torch.bfloat16: _lib.OUT_BF16, torch.float16: _lib.OUT_F16}
_FP4_STORAGE = tuple(d for d in (getattr(torch, "float4_e2m1fn_x2", None), torch.uint8) if d is not None)
_E8M0_STORAGE = tuple(d for d in (getattr(torch, "float8_e8m0fnu", None), torch.uint8) if d is not None)
_MAX_M, _MAX_N, _MAX_K = 2**20, 262144, 65536
_OOC = FallbackReason.OUT_OF_CONTRACT
_BLOCK = (128, 128)


def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _out_dtype(out, out_dtype):
    """The output dtype, or None when out and out_dtype disagree or it is not bf16/fp16."""
    if out is not None:
        if out_dtype is not None and out_dtype != out.dtype:
            return None
        dt = out.dtype
    else:
        dt = torch.bfloat16 if out_dtype is None else out_dtype
    return dt if dt in _OUT else None


def _out_ok(out, m, n, dtype, device, inputs) -> bool:
    if out is None:
        return True
    if not isinstance(out, torch.Tensor) or tuple(out.shape) != (m, n) or out.dtype != dtype:
        return False
    if out.device != device or not out.is_contiguous() or not aligned(out):
        return False
    return not any(overlaps(out, t) for t in inputs if t is not None)


@dataclass
class _Gemm8Plan:
    a: torch.Tensor
    b: torch.Tensor
    a_scale: torch.Tensor
    b_scale: torch.Tensor
    bias: torch.Tensor | None
    out: torch.Tensor | None
    out_dtype: torch.dtype
    m: int
    n: int
    k: int
    sa_sm: int
    sa_sk: int
    b_layout: int
    variant: str
    kernel_ref: str = field(default="")
    transpose_b: bool = False  # b is (k, n): transposed into (n, k) scratch first


def _run_gemm8(p: _Gemm8Plan):
    dev = p.a.device
    out = p.out if p.out is not None else torch.empty((p.m, p.n), dtype=p.out_dtype, device=dev)
    L = _lib.lib()
    b = p.b
    if p.transpose_b:
        b = torch.empty((p.n, p.k), dtype=p.b.dtype, device=dev)
        _lib.check(L.aklr_transpose_b8(p.b.data_ptr(), p.k, p.n, p.b.stride(0), b.data_ptr(), p.k, _stream(dev)),
                   "gemm_a8w8_blockwise_scaled (b transpose)")
    ws_bytes = L.aklr_gemm_a8w8_blockscale_workspace_bytes(p.m, p.n, p.k)
    ws = workspace.get(dev, ws_bytes)
    st = L.aklr_gemm_a8w8_blockscale(
        p.a.data_ptr(), p.a.stride(0), b.data_ptr(), b.stride(0) if p.b_layout == _lib.B_ROW_MAJOR else p.k,
        p.a_scale.data_ptr(), p.sa_sm, p.sa_sk, p.b_scale.data_ptr(), p.b_scale.stride(0),
        p.bias.data_ptr() if p.bias is not None else None, out.data_ptr(), out.stride(0), p.m, p.n, p.k,
        _FP8[p.a.dtype], p.b_layout, _OUT[p.out_dtype], ws.data_ptr() if ws is not None else None, ws_bytes,
        _stream(dev),
    )
    _lib.check(st, "gemm_a8w8_blockwise_scaled")
    return out


@api("gemm_a8w8_blockwise_scaled@1.0", _run_gemm8)
def gemm_a8w8_blockwise_scaled(
    a,
    b,
    a_scale,
    b_scale,
    block_size=_BLOCK,
    scale_major_mode="K",
    trans_b=True,
    bias=None,
    out_dtype=None,
    out=None,
    *,
    operand_format="none:none",
):
    # api-only parameter: anything but the default is out of contract (_dispatcher.py:301-309)
    if block_size is not _BLOCK and block_size != _BLOCK:
        return _OOC
    tensors = (a, b, a_scale, b_scale)
    if not all(isinstance(t, torch.Tensor) for t in tensors) or (bias is not None and not isinstance(bias, torch.Tensor)):
        return _OOC
    if scale_major_mode not in ("K", "MN") or trans_b not in (True, False):
        return _OOC
    # layout variant (contract.py:280-307)
    b_shuffled = getattr(b, "is_shuffled", False) is True
    sa_row_major = getattr(a_scale, "is_row_major", False) is True
    if operand_format == "none:none" and not b_shuffled:
        variant = "row_major"
    elif operand_format == "none:preshuffled":
        variant = "b_shuffled_row_major_a_scale" if sa_row_major else "b_shuffled"
    else:
        return _OOC
    if variant != "row_major" and not (trans_b and scale_major_mode == "K" and bias is None
                                       and a.dtype == torch.float8_e4m3fn):
        return _OOC
    # dtypes
    if a.dtype not in _FP8 or b.dtype != a.dtype or a_scale.dtype != torch.float32 or b_scale.dtype != torch.float32:
        return _OOC
    if bias is not None and bias.dtype != torch.float32:
        return _OOC
    dt = _out_dtype(out, out_dtype)
    if dt is None:
        return _OOC
    # shapes
    if a.dim() != 2 or b.dim() != 2 or a_scale.dim() != 2 or b_scale.dim() != 2:
        return _OOC
    m, k = a.shape
    n = b.shape[0] if trans_b else b.shape[1]
    if (b.shape[1] if trans_b else b.shape[0]) != k:
        return _OOC
    if not (1 <= m <= _MAX_M and 16 <= n <= _MAX_N and n % 16 == 0 and 128 <= k <= _MAX_K and k % 128 == 0):
        return _OOC
    kb = k // 128
    # a_scale storage: K-major (m, kb) / MN-major (kb, m) row-major; ColumnMajor for b_shuffled
    if variant == "b_shuffled":
        if tuple(a_scale.shape) != (m, kb):
            return _OOC
        if a_scale.is_contiguous():
            sa_sm, sa_sk = 1, m  # the transpose's bytes viewed as (m, kb)
        elif a_scale.mT.is_contiguous():
            a_scale = a_scale.mT.reshape(a_scale.shape)  # the view rewrite of ColumnMajor (_layouts.py:98-100)
            sa_sm, sa_sk = 1, m
        else:
            return _OOC
    else:
        want = (m, kb) if scale_major_mode == "K" else (kb, m)
        if tuple(a_scale.shape) != want or not a_scale.is_contiguous():
            return _OOC
        sa_sm, sa_sk = (kb, 1) if scale_major_mode == "K" else (1, m)
    if tuple(b_scale.shape) != (-(-n // 128), kb) or not b_scale.is_contiguous():
        return _OOC
    if bias is not None and (tuple(bias.shape) != (n,) or not bias.is_contiguous()):
        return _OOC
    if not a.is_contiguous() or not b.is_contiguous():
        return _OOC
    # device, alignment, overlap
    if not on_gpu(a, b, a_scale, b_scale, bias, out):
        return _OOC
    if not all(aligned(t) for t in (a, b, a_scale, b_scale) + ((bias,) if bias is not None else ())):
        return _OOC
    if not _out_ok(out, m, n, dt, a.device, (a, b, a_scale, b_scale, bias)):
        return _OOC
    b_layout = _lib.B_ROW_MAJOR if variant == "row_major" else _lib.B_PRESHUFFLE_16x16
    path = ("stream", "lds")[_lib.lib().aklr_gemm_a8w8_blockscale_kernel(m, n, k, b_layout)]  # as the library picks
    # trans_b = False (row_major only, by the check above): b is (k, n), as the reference's _weight
    # transposes it (aklr/ops/gemm/reference.py:32-37)
    ref = f"aklr_gemm_a8w8_blockscale:{path}" if trans_b else f"aklr_transpose_b8+aklr_gemm_a8w8_blockscale:{path}"
    return _Gemm8Plan(a, b, a_scale, b_scale, bias, out, dt, m, n, k, sa_sm, sa_sk, b_layout, variant, ref,
                      transpose_b=not trans_b)


# ---------------------------------------------------------------------------------------------
@dataclass
class _QuantGemm8Plan:
    x: torch.Tensor
    b: torch.Tensor
    b_scale: torch.Tensor
    bias: torch.Tensor | None
    out: torch.Tensor | None
    out_dtype: torch.dtype
    m: int
    n: int
    k: int
    b_layout: int
    variant: str
    kernel_ref: str = field(default="")


def _run_quant_gemm8(p: _QuantGemm8Plan):
    dev = p.x.device
    out = p.out if p.out is not None else torch.empty((p.m, p.n), dtype=p.out_dtype, device=dev)
    L = _lib.lib()
    ws_bytes = L.aklr_quant_gemm_a8w8_blockscale_workspace_bytes(p.m, p.n, p.k)
    ws = workspace.get(dev, ws_bytes)
    st = L.aklr_quant_gemm_a8w8_blockscale(
        p.x.data_ptr(), p.x.stride(0), p.b.data_ptr(), p.b.stride(0) if p.b_layout == _lib.B_ROW_MAJOR else p.k,
        p.b_scale.data_ptr(), p.b_scale.stride(0), p.bias.data_ptr() if p.bias is not None else None,
        out.data_ptr(), out.stride(0), p.m, p.n, p.k, p.b_layout, _OUT[p.out_dtype],
        ws.data_ptr() if ws is not None else None, ws_bytes, _stream(dev),
    )
    _lib.check(st, "quant_gemm_a8w8_blockwise_scaled")
    return out


@api("quant_gemm_a8w8_blockwise_scaled@1.0", _run_quant_gemm8)
def quant_gemm_a8w8_blockwise_scaled(x, b, b_scale, bias=None, out_dtype=None, out=None, *,
                                     operand_format="none:none"):
    """``gemm_a8w8_blockwise_scaled(*per_group_quant_fp8(x), b, b_scale, ...)`` in one call, equal bit for
    bit: bf16 activations x [m, k] are quantized per 1 x 128 group (aklr/ops/quant/reference.py:9-28) and
    multiplied by the 128 x 128-block-scaled e4m3 weight (aklr/ops/gemm/reference.py:90-105). This is the
    pair of ops sglang's fp8 block-quant linear calls; for m <= 16 the GEMM's compute waves quantize each K
    block themselves (one launch, no codes or scales in HBM) wherever the GEMM's own plan sums in the same
    order (not on wave-split-K or long-K plans, which run the two kernels). b: e4m3fn [n, k] ("none:none") or aiter's 16x16
    preshuffled layout ("none:preshuffled"); b_scale fp32 [ceil(n/128), k/128]; bias fp32 [n] or None.
    Calls it does not serve return a ``FallbackReason``."""
    if not all(isinstance(t, torch.Tensor) for t in (x, b, b_scale)) or (bias is not None and not isinstance(bias, torch.Tensor)):
        return _OOC
    b_shuffled = getattr(b, "is_shuffled", False) is True
    if operand_format == "none:none" and not b_shuffled:
        variant, b_layout = "row_major", _lib.B_ROW_MAJOR
    elif operand_format == "none:preshuffled":
        variant, b_layout = "b_shuffled", _lib.B_PRESHUFFLE_16x16
    else:
        return _OOC
    if x.dtype != torch.bfloat16 or b.dtype != torch.float8_e4m3fn or b_scale.dtype != torch.float32:
        return _OOC
    if bias is not None and (bias.dtype != torch.float32 or bias.dim() != 1 or not bias.is_contiguous()):
        return _OOC
    dt = _out_dtype(out, out_dtype)
    if dt is None or x.dim() != 2 or b.dim() != 2 or b_scale.dim() != 2:
        return _OOC
    m, k = x.shape
    n = b.shape[0]
    if b.shape[1] != k or not (1 <= m <= _MAX_M and 16 <= n <= _MAX_N and n % 16 == 0 and 128 <= k <= _MAX_K
                               and k % 128 == 0):
        return _OOC
    if tuple(b_scale.shape) != (-(-n // 128), k // 128) or not b_scale.is_contiguous():
        return _OOC
    if bias is not None and tuple(bias.shape) != (n,):
        return _OOC
    if x.stride(1) != 1 or x.stride(0) < k or x.stride(0) % 8 != 0 or not b.is_contiguous():
        return _OOC
    if not on_gpu(x, b, b_scale, bias, out):
        return _OOC
    if not all(aligned(t) for t in (x, b, b_scale) + ((bias,) if bias is not None else ())):
        return _OOC
    if not _out_ok(out, m, n, dt, x.device, (x, b, b_scale, bias)):
        return _OOC
    fused = _lib.lib().aklr_quant_gemm_a8w8_blockscale_fused(m, n, k) == 1  # as the library picks
    path = "stream_fused" if fused else ("stream", "lds")[_lib.lib().aklr_gemm_a8w8_blockscale_kernel(m, n, k, b_layout)]
    return _QuantGemm8Plan(x, b, b_scale, bias, out, dt, m, n, k, b_layout, variant,
                           f"aklr_quant_gemm_a8w8_blockscale:{path}")


# ---------------------------------------------------------------------------------------------
@dataclass
class _Gemm4Plan:
    a: torch.Tensor
    b: torch.Tensor
    a_scale: torch.Tensor
    b_scale: torch.Tensor
    bias: torch.Tensor | None
    out: torch.Tensor | None
    out_dtype: torch.dtype
    m: int
    n: int
    k: int
    b_layout: int
    scale_layout: int
    variant: str
    kernel_ref: str = field(default="")


def _u8(t):
    return t if t.dtype == torch.uint8 else t.view(torch.uint8)


def _run_gemm4(p: _Gemm4Plan):
    dev = p.a.device
    out = p.out if p.out is not None else torch.empty((p.m, p.n), dtype=p.out_dtype, device=dev)
    L = _lib.lib()
    ws_bytes = L.aklr_gemm_a4w4_mxfp4_workspace_bytes(p.m, p.n, p.k)
    ws = workspace.get(dev, ws_bytes)
    a, b, sa, sb = _u8(p.a), _u8(p.b), _u8(p.a_scale), _u8(p.b_scale)
    st = L.aklr_gemm_a4w4_mxfp4(
        a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0), sa.data_ptr(), sa.stride(0), sb.data_ptr(),
        sb.stride(0), p.bias.data_ptr() if p.bias is not None else None, out.data_ptr(), out.stride(0), p.m,
        p.n, p.k, p.b_layout, p.scale_layout, _OUT[p.out_dtype], ws.data_ptr() if ws is not None else None,
        ws_bytes, _stream(dev),
    )
    _lib.check(st, "gemm_a4w4_mxfp4")
    return out


@api("gemm_a4w4_mxfp4@1.0", _run_gemm4)
def gemm_a4w4_mxfp4(
    a,
    b,
    a_scale,
    b_scale,
    alpha=1.0,
    beta=0.0,
    trans_b=True,
    bias=None,
    out_dtype=None,
    out=None,
    *,
    operand_format="none:preshuffled",
):
    tensors = (a, b, a_scale, b_scale)
    if not all(isinstance(t, torch.Tensor) for t in tensors) or (bias is not None and not isinstance(bias, torch.Tensor)):
        return _OOC
    # ScalarSpec values: alpha (1.0,), beta (0.0,); trans_b True only (contract.py:342-352)
    if alpha != 1.0 or beta != 0.0 or trans_b is not True:
        return _OOC
    if operand_format == "none:none":
        variant = "row_major"
    elif operand_format == "none:preshuffled":
        variant = "b_shuffled"
    else:
        return _OOC
    if a.dtype not in _FP4_STORAGE or b.dtype not in _FP4_STORAGE:
        return _OOC
    if a_scale.dtype not in _E8M0_STORAGE or b_scale.dtype not in _E8M0_STORAGE:
        return _OOC
    if bias is not None and bias.dtype != torch.float32:
        return _OOC
    dt = _out_dtype(out, out_dtype)
    if dt is None:
        return _OOC
    if a.dim() != 2 or b.dim() != 2 or a_scale.dim() != 2 or b_scale.dim() != 2:
        return _OOC
    m, kh = a.shape
    n = b.shape[0]
    k = 2 * kh
    if b.shape[1] != kh:
        return _OOC
    if not (1 <= m <= _MAX_M and 16 <= n <= _MAX_N and n % 16 == 0 and 64 <= k <= _MAX_K and k % 64 == 0):
        return _OOC
    g = k // 32
    if variant == "row_major":
        sa_shape, sb_shape = (m, g), (n, g)
    else:
        sa_shape = (-(-m // 256) * 256, -(-g // 8) * 8)
        sb_shape = (-(-n // 256) * 256, -(-g // 8) * 8)
    if tuple(a_scale.shape) != sa_shape or tuple(b_scale.shape) != sb_shape:
        return _OOC
    if not all(t.is_contiguous() for t in tensors):
        return _OOC
    if bias is not None and (tuple(bias.shape) != (n,) or not bias.is_contiguous()):
        return _OOC
    if not on_gpu(a, b, a_scale, b_scale, bias, out):
        return _OOC
    if not all(aligned(t) for t in tensors + ((bias,) if bias is not None else ())):
        return _OOC
    if not _out_ok(out, m, n, dt, a.device, (a, b, a_scale, b_scale, bias)):
        return _OOC
    pre = variant == "b_shuffled"
    path = "skinny" if m <= 16 else ("stream" if m <= 32 else "lds")  # as the library picks (aligned scales)
    return _Gemm4Plan(a, b, a_scale, b_scale, bias, out, dt, m, n, k,
                      _lib.B_PRESHUFFLE_16x16 if pre else _lib.B_ROW_MAJOR,
                      _lib.SCALES_SHUFFLED if pre else _lib.SCALES_ROW_MAJOR, variant,
                      f"aklr_gemm_a4w4_mxfp4:{path}")

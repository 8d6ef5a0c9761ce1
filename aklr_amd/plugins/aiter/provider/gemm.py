# SPDX-License-Identifier: MIT
# Copyright (C) 2026, Advanced Micro Devices, Inc. All rights reserved.
# The host protocol and rules here follow aklr/plugins/aiter/provider/gemm.py, whose licence notice this is.

"""aiter's fp8 GEMMs with a fp32 scale per 128 x 128 of the weight and per 1 x 128 of the
activations, served by ``gemm_a8w8_blockwise_scaled`` (aklr/plugins/aiter/provider/gemm.py:30-96).

aiter keeps each weight layout as its own op; here they are operand formats of one op:

- ``gemm_a8w8_blockscale(xq, wq, x_scale, w_scale, dtype, is_b_preshuffled, split_k)``: row-major
  weight, K-major x_scale. Declines a preshuffled weight, any ``split_k`` and non-fp32 scales.
- ``gemm_a8w8_blockscale_bpreshuffle(xq, wq, x_scale, w_scale, dtype, out)``: 16x16-shuffled weight,
  x_scale holding aiter's column-major bytes (operand_format "none:preshuffled"). Declines an
  x_scale marked ``is_row_major`` (aiter would read its bytes column-major).
- ``gemm_a8w8_blockscale_out(x, w, x_scale, w_scale, dtype, y, config, skip_reduce, kernel_type)``:
  row-major, result into ``y`` when given; ``config``/``kernel_type`` only pick aiter's schedule.
  Declines ``skip_reduce`` and a non-contiguous x_scale.
"""
from __future__ import annotations

import torch

from ....gemm import gemm_a8w8_blockwise_scaled
from ._base import offer, selector, served


def _fp32_scales(x_scale, w_scale) -> bool:
    return x_scale.dtype == torch.float32 and w_scale.dtype == torch.float32


def _out_dtype(dtype, y):
    return dtype if y is None else y.dtype


@selector("gemm_a8w8_blockscale")
def _select_gemm_a8w8_blockscale(args, kwargs):
    xq, wq, x_scale, w_scale, dtype, is_b_preshuffled, split_k = args
    if is_b_preshuffled or split_k is not None or not _fp32_scales(x_scale, w_scale):
        return None
    return offer(gemm_a8w8_blockwise_scaled.serving(xq, wq, x_scale, w_scale, out_dtype=dtype),
                 _run_gemm_a8w8_blockscale)


def _run_gemm_a8w8_blockscale(xq, wq, x_scale, w_scale, dtype, is_b_preshuffled, split_k):
    return served(gemm_a8w8_blockwise_scaled(xq, wq, x_scale, w_scale, out_dtype=dtype))


@selector("gemm_a8w8_blockscale_bpreshuffle")
def _select_gemm_a8w8_blockscale_bpreshuffle(args, kwargs):
    xq, wq, x_scale, w_scale, dtype, out = args
    if not _fp32_scales(x_scale, w_scale) or getattr(x_scale, "is_row_major", False):
        return None
    return offer(
        gemm_a8w8_blockwise_scaled.serving(xq, wq, x_scale, w_scale, out_dtype=dtype, out=out,
                                           operand_format="none:preshuffled"),
        _run_gemm_a8w8_blockscale_bpreshuffle,
    )


def _run_gemm_a8w8_blockscale_bpreshuffle(xq, wq, x_scale, w_scale, dtype, out):
    return served(gemm_a8w8_blockwise_scaled(xq, wq, x_scale, w_scale, out_dtype=dtype, out=out,
                                             operand_format="none:preshuffled"))


@selector("gemm_a8w8_blockscale_out")
def _select_gemm_a8w8_blockscale_out(args, kwargs):
    x, w, x_scale, w_scale, dtype, y, config, skip_reduce, kernel_type = args
    if (skip_reduce or _out_dtype(dtype, y) is None or not _fp32_scales(x_scale, w_scale)
            or not x_scale.is_contiguous()):
        return None
    return offer(
        gemm_a8w8_blockwise_scaled.serving(x, w, x_scale, w_scale, out_dtype=_out_dtype(dtype, y), out=y,
                                           operand_format="none:none"),
        _run_gemm_a8w8_blockscale_out,
    )


def _run_gemm_a8w8_blockscale_out(x, w, x_scale, w_scale, dtype, y, config, skip_reduce, kernel_type):
    return served(gemm_a8w8_blockwise_scaled(x, w, x_scale, w_scale, out_dtype=_out_dtype(dtype, y), out=y,
                                             operand_format="none:none"))

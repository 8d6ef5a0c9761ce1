"""CPU oracle for the block-scaled FP8 / MXFP4 GEMM path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic the reference (AMD-AGI/AKLR) defines for the path:

- ``quant``:   per_group_quant_fp8 (aklr/ops/quant/reference.py:9-28), per_group_quant_mxfp8
               (aklr/ops/quant/reference.py:31-48) and the MXFP4 activation quantizer ``_mxfp4``
               (aklr/ops/fused_moe/reference.py:21-37);
- ``gemm``:    gemm_a8w8_blockwise_scaled (aklr/ops/gemm/reference.py:90-105) and gemm_a4w4_mxfp4
               (aklr/ops/gemm/reference.py:108-122);
- ``formats``: the element decodings (aklr/core/contract/semantics/_dtypes.py:55-110) and e4m3/e2m1
               rounding;
- ``layouts``: Preshuffle / ColumnMajor / E8M0Scales (aklr/core/contract/semantics/_layouts.py:20-156);
- ``moe``:     the grouped DeepSeek FP8 MoE (aklr/plugins/sglang/models/deepseek_v2/reference.py:121-183).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it, and
only as the checker (or as the timed CPU baseline). The product (``aklr_amd``) never imports it: the
GPU path has no CPU fallback.

How each function is pinned (none of the reference's tests holds golden vectors for this path):
see the header of each module; every function has at least one check in ``tests/test_oracle_*.py``
that a plausible mistake (a dropped term, a wrong sign or index, a transposed operand) would fail.
"""

"""Host logic of the op APIs without a GPU: what each call is served as, or why it falls back
(FallbackReason values of aklr/core/runtime/dispatch/_dispatcher.py:53-70), with the device check
switched off so CPU tensors stand in for GPU ones (nothing is launched: only ``serving`` and
``fallback_reason`` are called, plus real calls on CPU tensors, which must fall back)."""
from __future__ import annotations

import pytest
import torch

import aklr_amd
from aklr_amd import FallbackReason as FR
from aklr_amd import gemm as hg
from aklr_amd import layouts
from aklr_amd import quant as hq


@pytest.fixture
def as_gpu(monkeypatch, native_lib):
    monkeypatch.setattr(hq, "on_gpu", lambda *t: True)
    monkeypatch.setattr(hg, "on_gpu", lambda *t: True)


def fp8(shape, dtype=torch.float8_e4m3fn):
    return torch.zeros(shape, dtype=torch.uint8).view(dtype)


def test_cpu_tensors_fall_back_never_raise():
    x = torch.zeros((4, 256), dtype=torch.bfloat16)
    assert aklr_amd.per_group_quant_fp8(x) is FR.OUT_OF_CONTRACT
    assert aklr_amd.per_group_quant_mxfp8(x) is FR.OUT_OF_CONTRACT
    assert aklr_amd.dynamic_mxfp4_quant(x) is FR.OUT_OF_CONTRACT
    a, b = fp8((4, 256)), fp8((16, 256))
    sa, sb = torch.ones((4, 2)), torch.ones((1, 2))
    assert aklr_amd.gemm_a8w8_blockwise_scaled(a, b, sa, sb) is FR.OUT_OF_CONTRACT
    assert aklr_amd.gemm_a8w8_blockwise_scaled.fallback_reason(a, b, sa, sb) is FR.OUT_OF_CONTRACT


def test_disable_env(monkeypatch, as_gpu):
    x = torch.zeros((4, 256), dtype=torch.bfloat16)
    monkeypatch.setenv("AKLR_DISABLE", "1")
    assert aklr_amd.per_group_quant_fp8.serving(x) is FR.DISABLED
    monkeypatch.setenv("AKLR_DISABLE", "gemm_a8w8_blockwise_scaled@1.0, per_group_quant_mxfp8@1.0")
    assert aklr_amd.per_group_quant_mxfp8.serving(x) is FR.DISABLED
    info = aklr_amd.per_group_quant_fp8.serving(x)
    assert info.contract_id == "per_group_quant_fp8@1.0" and info.kernel_ref == "aklr_per_group_quant_fp8"
    monkeypatch.setenv("AKLR_DISABLE", "0")
    assert not isinstance(aklr_amd.per_group_quant_mxfp8.serving(x), FR)


def test_trace_env_rejects_bad_value(monkeypatch, as_gpu):
    monkeypatch.setenv("AKLR_TRACE", "verbose")
    with pytest.raises(ValueError):
        aklr_amd.per_group_quant_fp8.serving(torch.zeros((1, 128), dtype=torch.bfloat16))
    monkeypatch.setenv("AKLR_TRACE", "op")
    assert not isinstance(aklr_amd.per_group_quant_fp8.serving(torch.zeros((1, 128), dtype=torch.bfloat16)), FR)


def test_quant_contract(as_gpu):
    ok = torch.zeros((3, 256), dtype=torch.bfloat16)
    assert not isinstance(aklr_amd.per_group_quant_fp8.serving(ok), FR)
    assert aklr_amd.per_group_quant_fp8.serving(torch.zeros((3, 192), dtype=torch.bfloat16)) is FR.OUT_OF_CONTRACT
    assert aklr_amd.per_group_quant_fp8.serving(torch.zeros((3, 256), dtype=torch.float16)) is FR.OUT_OF_CONTRACT
    assert aklr_amd.per_group_quant_fp8.serving(torch.zeros((256, 3), dtype=torch.bfloat16).t()) is FR.OUT_OF_CONTRACT
    assert aklr_amd.per_group_quant_fp8.serving(torch.zeros((2, 21504 + 128), dtype=torch.bfloat16)) is FR.OUT_OF_CONTRACT
    assert not isinstance(aklr_amd.per_group_quant_mxfp8.serving(torch.zeros((3, 96), dtype=torch.bfloat16)), FR)
    s = aklr_amd.dynamic_mxfp4_quant.serving(torch.zeros((3, 96), dtype=torch.bfloat16), shuffle=True)
    assert s.variant == "shuffled_scales"


def _g8(m=4, n=144, k=256, **kw):
    a, b = fp8((m, k)), fp8((n, k))
    sa, sb = torch.ones((m, k // 128)), torch.ones((-(-n // 128), k // 128))
    return a, b, sa, sb


def test_gemm8_variants(as_gpu):
    a, b, sa, sb = _g8()
    s = aklr_amd.gemm_a8w8_blockwise_scaled.serving(a, b, sa, sb)
    assert s.variant == "row_major" and s.kernel_ref.endswith(":stream")
    assert aklr_amd.gemm_a8w8_blockwise_scaled.serving(fp8((300, 256)), b, torch.ones((300, 2)), sb).kernel_ref.endswith(":lds")
    # MN-major a_scale
    assert not isinstance(aklr_amd.gemm_a8w8_blockwise_scaled.serving(a, b, sa.t().contiguous(), sb,
                                                                      scale_major_mode="MN"), FR)
    # preshuffled weight with column-major a_scale (the group-major bytes), and its (1, m)-strided view
    bs = layouts.shuffle_weight(b)
    sa_cm = layouts.column_major(sa)
    s = aklr_amd.gemm_a8w8_blockwise_scaled.serving(a, bs, sa_cm, sb, operand_format="none:preshuffled")
    assert s.variant == "b_shuffled"
    s = aklr_amd.gemm_a8w8_blockwise_scaled.serving(a, bs, sa.t().contiguous().mT, sb, operand_format="none:preshuffled")
    assert s.variant == "b_shuffled"
    sa_rm = sa.clone()
    sa_rm.is_row_major = True
    s = aklr_amd.gemm_a8w8_blockwise_scaled.serving(a, bs, sa_rm, sb, operand_format="none:preshuffled")
    assert s.variant == "b_shuffled_row_major_a_scale"
    # a shuffled weight in the row_major format is no variant
    assert aklr_amd.gemm_a8w8_blockwise_scaled.serving(a, bs, sa, sb) is FR.OUT_OF_CONTRACT


def test_gemm8_out_of_contract(as_gpu):
    a, b, sa, sb = _g8()
    api = aklr_amd.gemm_a8w8_blockwise_scaled.serving
    assert api(a, b, sa, sb, block_size=(64, 64)) is FR.OUT_OF_CONTRACT  # api-only parameter off default
    # the reference's guard compares with != against the default tuple: a list is out of contract
    assert api(a, b, sa, sb, block_size=[128, 128]) is FR.OUT_OF_CONTRACT
    assert api(a, b, sa, sb, block_size=(128, 128)) is not FR.OUT_OF_CONTRACT
    assert api(a, fp8((144, 256), torch.float8_e5m2), sa, sb) is FR.OUT_OF_CONTRACT  # mixed fp8 dtypes
    assert api(a, b, sa.double(), sb) is FR.OUT_OF_CONTRACT
    assert api(a, b, sa[:, :1], sb) is FR.OUT_OF_CONTRACT  # wrong a_scale shape
    assert api(a, fp8((136, 256)), sa, sb) is FR.OUT_OF_CONTRACT  # n % 16
    assert api(fp8((4, 200)), fp8((144, 200)), sa, sb) is FR.OUT_OF_CONTRACT  # k % 128
    assert api(a, b, sa, sb, out_dtype=torch.float32) is FR.OUT_OF_CONTRACT
    bias = torch.zeros(144)
    bs = layouts.shuffle_weight(b)
    assert api(a, bs, layouts.column_major(sa), sb, bias=bias, operand_format="none:preshuffled") is FR.OUT_OF_CONTRACT
    assert api(a, b, sa, sb, operand_format="none:bogus") is FR.OUT_OF_CONTRACT
    out = torch.empty((4, 144), dtype=torch.bfloat16)
    assert not isinstance(api(a, b, sa, sb, out=out), FR)
    assert api(a, b, sa, sb, out=out, out_dtype=torch.float16) is FR.OUT_OF_CONTRACT
    assert api(a, b, sa, sb, out=torch.empty((4, 143), dtype=torch.bfloat16)) is FR.OUT_OF_CONTRACT
    # output overlapping an input
    big = torch.empty(4 * 144 * 2 + 4096, dtype=torch.uint8)
    aa = big[: 4 * 256].view(torch.float8_e4m3fn).view(4, 256)
    oo = big[:4 * 144 * 2].view(torch.bfloat16).view(4, 144)
    assert api(aa, b, sa, sb, out=oo) is FR.OUT_OF_CONTRACT
    # trans_b=False (b as (k, n)) is served on row_major: b transposed first, then the same GEMM
    plan = api(a, fp8((256, 144)), sa, sb, trans_b=False)
    assert not isinstance(plan, FR) and plan.kernel_ref.startswith("aklr_transpose_b8+aklr_gemm_a8w8_blockscale")
    assert api(a, fp8((144, 256)), sa, sb, trans_b=False) is FR.OUT_OF_CONTRACT  # (n, k) given for (k, n)
    # the shuffled variants take trans_b only (contract.py:242-246)
    assert api(a, layouts.shuffle_weight(fp8((144, 256))), layouts.column_major(sa), sb, trans_b=False,
               operand_format="none:preshuffled") is FR.OUT_OF_CONTRACT


def test_gemm4_variants(as_gpu):
    m, n, k = 4, 32, 192
    a = torch.zeros((m, k // 2), dtype=torch.uint8)
    b = torch.zeros((n, k // 2), dtype=torch.uint8)
    sa = torch.zeros((m, k // 32), dtype=torch.uint8)
    sb = torch.zeros((n, k // 32), dtype=torch.uint8)
    api = aklr_amd.gemm_a4w4_mxfp4.serving
    assert api(a, b, sa, sb, operand_format="none:none").variant == "row_major"
    # the default format is the preshuffled one, whose scales are padded and shuffled
    assert api(a, b, sa, sb) is FR.OUT_OF_CONTRACT
    s = api(a, layouts.shuffle_weight(b), layouts.e8m0_scales(sa), layouts.e8m0_scales(sb))
    assert s.variant == "b_shuffled"
    assert api(a, b, sa, sb, alpha=2.0, operand_format="none:none") is FR.OUT_OF_CONTRACT
    assert api(a, b, sa, sb, beta=1.0, operand_format="none:none") is FR.OUT_OF_CONTRACT
    assert api(torch.zeros((m, 40), dtype=torch.uint8), torch.zeros((n, 40), dtype=torch.uint8),
               torch.zeros((m, 2), dtype=torch.uint8), torch.zeros((n, 2), dtype=torch.uint8),
               operand_format="none:none") is FR.OUT_OF_CONTRACT  # k = 80, not a multiple of 64


# ---------------------------------------------------------------------------------------------
# deepseek_v2_fp8_moe (deepseek_v2/contract.py:188-320)
def _moe_args(t=4, n_routed=16, d=256, inter=128, shuffled=False):
    from aklr_amd import layouts as lay

    bf = torch.bfloat16
    w1, w2 = fp8((n_routed + 1, 2 * inter, d)), fp8((n_routed + 1, d, inter))
    if shuffled:
        w1, w2 = lay.shuffle_weight(w1), lay.shuffle_weight(w2)
    return [torch.zeros((t, d), dtype=bf), torch.zeros((n_routed, d), dtype=bf), torch.zeros((n_routed,), dtype=bf),
            w1, torch.ones((n_routed + 1, 2 * inter // 128, d // 128)), w2,
            torch.ones((n_routed + 1, d // 128, inter // 128)), 8, 8, 4, True, "sigmoid", 2.5]


@pytest.fixture
def moe_as_gpu(monkeypatch, native_lib):
    from aklr_amd import moe as hm

    monkeypatch.setattr(hm, "on_gpu", lambda *t: True)


def test_moe_serving_and_variants(moe_as_gpu):
    info = aklr_amd.deepseek_v2_fp8_moe.serving(*_moe_args())
    assert info.contract_id == "deepseek_v2_fp8_moe@1.0" and info.variant == "row_major"
    assert aklr_amd.deepseek_v2_fp8_moe.serving(*_moe_args(shuffled=True)).variant == "shuffled_16x16"
    glm = _moe_args(n_routed=32)
    glm[8], glm[9] = 1, 1
    assert not isinstance(aklr_amd.deepseek_v2_fp8_moe.serving(*glm), FR)


@pytest.mark.parametrize("index,value", [(7, 6), (8, 4), (9, 2), (10, False), (11, "softmax"), (12, 1.0)])
def test_moe_attrs_outside_contract(moe_as_gpu, index, value):
    args = _moe_args()
    args[index] = value
    assert aklr_amd.deepseek_v2_fp8_moe.fallback_reason(*args) is FR.OUT_OF_CONTRACT


def test_moe_shapes_and_layouts_outside_contract(moe_as_gpu):
    args = _moe_args()
    args[0] = torch.zeros((4, 200), dtype=torch.bfloat16)  # model_dim % 128
    assert aklr_amd.deepseek_v2_fp8_moe.fallback_reason(*args) is FR.OUT_OF_CONTRACT
    args = _moe_args()
    args[3].is_shuffled = True  # w1 shuffled, w2 not: no variant
    assert aklr_amd.deepseek_v2_fp8_moe.fallback_reason(*args) is FR.OUT_OF_CONTRACT
    args = _moe_args(n_routed=12)  # 12 experts in 8 groups
    assert aklr_amd.deepseek_v2_fp8_moe.fallback_reason(*args) is FR.OUT_OF_CONTRACT
    args = _moe_args()
    args[4] = torch.ones((17, 1, 2))  # w1_scale rows
    assert aklr_amd.deepseek_v2_fp8_moe.fallback_reason(*args) is FR.OUT_OF_CONTRACT


def test_moe_cpu_tensors_fall_back():
    assert aklr_amd.deepseek_v2_fp8_moe(*_moe_args()) is FR.OUT_OF_CONTRACT


def test_moe_workspace_bytes(native_lib):
    # DeepSeek-V3 at T=4096: [T, 7168] fp8 codes, 9 slots of h and y, and the small tables
    b = native_lib.aklr_moe_fp8_workspace_bytes(4096, 7168, 2048, 257, 9, 256)
    r = 4096 * 9
    assert b >= r * 7168 * 2 + r * 2048 + 4096 * 7168
    assert native_lib.aklr_moe_fp8_workspace_bytes(4096, 7000, 2048, 257, 9, 256) == 0


def test_moe_large_token_counts_are_served_in_chunks(moe_as_gpu, native_lib):
    # In contract up to 65536 tokens; the kernels' 32-bit offsets take fewer per call at D=7168 (9 slots:
    # R * D * 2 < 2**31 -> 16644 tokens). serving() says served, and the host runs the call as chunks the
    # library takes, each with a workspace it sizes (so the call cannot raise for its size).
    from aklr_amd import moe as hm

    d, inter, slots = 7168, 2048, 9
    for tokens in (1, 4096, 16644, 16645, 32768, 65536):
        chunks = hm.token_chunks(tokens, d, inter, slots)
        assert chunks[0][0] == 0 and chunks[-1][1] == tokens
        assert all(a < b and b == c for (a, b), (c, _) in zip(chunks, chunks[1:] + [(tokens, 0)]))
        for a, b in chunks:
            assert native_lib.aklr_moe_fp8_workspace_bytes(b - a, d, inter, 257, slots, 256) > 0
        assert len(chunks) == -(-tokens // 16644)
    # the largest chunk is the library's own limit: one more token is refused
    assert native_lib.aklr_moe_fp8_workspace_bytes(16645, d, inter, 257, slots, 256) == 0
    args = _moe_args(t=32768, n_routed=16, d=7168, inter=128)
    assert not isinstance(aklr_amd.deepseek_v2_fp8_moe.serving(*args), FR)

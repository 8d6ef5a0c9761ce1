"""GPU checks of the scratch rule: no call depends on what the workspace held before it.

The reference's kernel ABI allocates scratch inside each call and never relies on earlier contents
(aklr/ops/README.md:214, :276-286). Here the split-K arrival words carry a tag of the launch, so a
workspace that is freshly allocated, filled with 0xFF, filled with random bytes, or left over from the
previous call of the same plan must give the same output, bit for bit, and that output must match the
oracle. Every case below runs a plan that splits K across workgroups (so the arrival words are used),
through the C ABI, on the stream, LDS and fused-quantization FP8 kernels and on the skinny, stream and
LDS MXFP4 kernels.

Graph replays: a captured call keeps its launch parameters but gets a new dispatch id on every replay;
each replay here runs on new inputs copied into the captured buffers, with eager work in between, and
must equal the eager call on the same inputs. Two graphs captured on one stream and replayed at the
same time on two streams each own their scratch (the per-call allocation comes from each graph's pool).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import aklr_amd
from aklr_amd import _lib, layouts, workloads
from oracle import gemm as ogemm
from tests.helpers import f32, say, u8

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _fills(nbytes: int, seed: int):
    """Workspace contents to start from: 0xFF everywhere, then random bytes."""
    g = workloads.generator(seed, DEV)
    yield "0xff", torch.full((nbytes,), 0xFF, dtype=torch.uint8, device=DEV)
    yield "random", torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=DEV, generator=g)


def _sample(m, n, rows=64, cols=512, seed=0):
    rng = np.random.default_rng(seed)
    r = np.arange(m) if m <= rows else np.sort(rng.choice(m, rows, replace=False))
    c = np.arange(n) if n <= cols else np.sort(rng.choice(n, cols, replace=False))
    return r, c


# FP8 plans that split K: stream kernel (m = 16 and 128 at 4 splits), LDS kernel with 128-row tiles
# split 4 ways (m = 256, n = 2112), the LDS 64-row tiles of a small output (64x64: m = 256, n = 512 at 40
# K blocks and m = 300, n = 1024 at 56; 64x128: m = 1000, n = 512 at 64 K blocks), and the stream
# kernel's row blocks split 2 ways (m = 100, n = 4096: 2 blocks).
FP8_SPLIT = [(16, 4096, 16384), (128, 2112, 7168), (256, 2112, 7168), (300, 1024, 7168),
             (100, 4096, 8192), (96, 576, 7168), (64, 2112, 7168), (50, 4096, 8192),
             (256, 512, 5120), (1000, 512, 8192)]


@pytest.mark.parametrize("m,n,k", FP8_SPLIT)
def test_fp8_gemm_any_workspace_content(m, n, k):
    L = _lib.lib()
    need = L.aklr_gemm_a8w8_blockscale_workspace_bytes(m, n, k)
    assert need > 131072, f"({m}, {n}, {k}) is expected to split K"
    say(f"fp8 gemm any-workspace m={m} n={n} k={k} ws={need}")
    x = workloads.activations(m, k, seed=m, device=DEV)
    q, s = aklr_amd.per_group_quant_fp8(x)  # s: [k/128, m] group-major = column-major a_scale
    b, bs = workloads.blockwise_fp8_weight(n, k, seed=m + 1, device=DEV)
    bb = layouts.shuffle_weight(b)
    outs = []

    def call(ws):
        out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
        st = L.aklr_gemm_a8w8_blockscale(q.data_ptr(), k, bb.data_ptr(), k, s.data_ptr(), 1, m, bs.data_ptr(),
                                         bs.stride(0), None, out.data_ptr(), n, m, n, k, _lib.FP8_E4M3FN,
                                         _lib.B_PRESHUFFLE_16x16, _lib.OUT_BF16, ws.data_ptr(), ws.numel(), _stream())
        assert st == 0, L.aklr_status_string(st)
        return out

    for name, ws in _fills(need, seed=m):
        outs.append((name, call(ws)))
        outs.append((name + "+leftover", call(ws)))  # the same buffer again: the previous call's words
    torch.cuda.synchronize()
    ref_out = outs[0][1]
    for name, o in outs:
        assert not torch.isnan(o.float()).any(), f"{name}: output not written"
        assert torch.equal(o.view(torch.int16), ref_out.view(torch.int16)), f"{name}: differs from the 0xff run"
    r, c = _sample(m, n, seed=m)
    ref = ogemm.gemm_a8w8_blockwise_scaled(u8(q), u8(b), s.cpu().numpy(), bs.cpu().numpy(), scale_major_mode="MN",
                                           rows=r, cols=c)
    got = f32(ref_out)[np.ix_(r, c)]
    assert ogemm.within_north_star(got, ref) and ogemm.within_contract_tolerance(got, ref)


@pytest.mark.parametrize("m,n,k", [(16, 4096, 16384), (4, 2112, 7168)])
def test_fused_quant_gemm_any_workspace_content(m, n, k):
    L = _lib.lib()
    assert L.aklr_quant_gemm_a8w8_blockscale_fused(m, n, k) == 1
    need = L.aklr_quant_gemm_a8w8_blockscale_workspace_bytes(m, n, k)
    say(f"fused quant gemm any-workspace m={m} n={n} k={k} ws={need}")
    x = workloads.activations(m, k, seed=m + 5, device=DEV)
    b, bs = workloads.blockwise_fp8_weight(n, k, seed=m + 6, device=DEV)
    bb = layouts.shuffle_weight(b)
    q, s = aklr_amd.per_group_quant_fp8(x)
    want = aklr_amd.gemm_a8w8_blockwise_scaled(q, bb, s.view(m, k // 128), bs, operand_format="none:preshuffled")
    for name, ws in _fills(max(need, 16), seed=m):
        for rep in range(2):
            out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
            st = L.aklr_quant_gemm_a8w8_blockscale(x.data_ptr(), k, bb.data_ptr(), k, bs.data_ptr(), bs.stride(0),
                                                   None, out.data_ptr(), n, m, n, k, _lib.B_PRESHUFFLE_16x16,
                                                   _lib.OUT_BF16, ws.data_ptr(), ws.numel(), _stream())
            assert st == 0
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"{name} call {rep}"


# MXFP4 plans that split K: skinny (m = 1, n = 2048: 64 column groups x 4 waves < 512, split 2), stream
# (m = 32, 10240 x 8192) and LDS with 128x128 tiles (m = 100, n = 272, k = 4096; m = 40, n = 2048).
MXFP4_SPLIT = [(1, 2048, 8192), (32, 10240, 8192), (100, 272, 4096), (40, 2048, 8192)]


@pytest.mark.parametrize("m,n,k", MXFP4_SPLIT)
def test_mxfp4_gemm_any_workspace_content(m, n, k):
    L = _lib.lib()
    need = L.aklr_gemm_a4w4_mxfp4_workspace_bytes(m, n, k)
    assert need > 131072, f"({m}, {n}, {k}) is expected to split K"
    say(f"mxfp4 gemm any-workspace m={m} n={n} k={k} ws={need}")
    x = workloads.activations(m, k, seed=m + 11, device=DEV)
    qa, sa = aklr_amd.dynamic_mxfp4_quant(x, shuffle=True)
    qa_rm, sa_rm = aklr_amd.dynamic_mxfp4_quant(x, shuffle=False)
    wb, sb = workloads.mxfp4_weight(n, k, seed=m + 12, device=DEV)
    wbs, sbs = layouts.shuffle_weight(wb), layouts.e8m0_scales(sb)
    a8, b8, sa8, sb8 = (t.view(torch.uint8) for t in (qa, wbs, sa, sbs))
    outs = []
    for name, ws in _fills(need, seed=m + 1):
        for rep in range(2):
            out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
            st = L.aklr_gemm_a4w4_mxfp4(a8.data_ptr(), k // 2, b8.data_ptr(), k // 2, sa8.data_ptr(), sa8.stride(0),
                                        sb8.data_ptr(), sb8.stride(0), None, out.data_ptr(), n, m, n, k,
                                        _lib.B_PRESHUFFLE_16x16, _lib.SCALES_SHUFFLED, _lib.OUT_BF16, ws.data_ptr(),
                                        ws.numel(), _stream())
            assert st == 0, L.aklr_status_string(st)
            outs.append((f"{name} call {rep}", out))
    torch.cuda.synchronize()
    for name, o in outs:
        assert not torch.isnan(o.float()).any(), f"{name}: output not written"
        assert torch.equal(o.view(torch.int16), outs[0][1].view(torch.int16)), name
    r, c = _sample(m, n, seed=m)
    ref = ogemm.gemm_a4w4_mxfp4(u8(qa_rm), u8(wb), u8(sa_rm), u8(sb), rows=r, cols=c)
    assert ogemm.within_north_star(f32(outs[0][1])[np.ix_(r, c)], ref)


def _decode_inputs(m, n, k, seed):
    x = workloads.activations(m, k, seed=seed, device=DEV)
    q, s = aklr_amd.per_group_quant_fp8(x)
    return q, s


def test_graph_replays_on_new_inputs():
    # decode FP8 (split K, stream kernel) and MXFP4 (split K, stream kernel) captured once, replayed four
    # times on new inputs with eager work between the replays; every replay equals the eager call
    m, n, k = 16, 4096, 16384
    b, bs = workloads.blockwise_fp8_weight(n, k, seed=3, device=DEV)
    bb = layouts.shuffle_weight(b)
    m4, n4, k4 = 32, 10240, 8192
    wb, sb = workloads.mxfp4_weight(n4, k4, seed=4, device=DEV)
    wbs, sbs = layouts.shuffle_weight(wb), layouts.e8m0_scales(sb)
    x8 = torch.empty((m, k), dtype=torch.bfloat16, device=DEV)
    x4 = torch.empty((m4, k4), dtype=torch.bfloat16, device=DEV)
    x8.copy_(workloads.activations(m, k, seed=100, device=DEV))
    x4.copy_(workloads.activations(m4, k4, seed=200, device=DEV))

    def step():
        q, s = aklr_amd.per_group_quant_fp8(x8)
        o8 = aklr_amd.gemm_a8w8_blockwise_scaled(q, bb, s.view(m, k // 128), bs, operand_format="none:preshuffled")
        qa, sa = aklr_amd.dynamic_mxfp4_quant(x4, shuffle=True)
        o4 = aklr_amd.gemm_a4w4_mxfp4(qa, wbs, sa, sbs)
        return o8, o4

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()  # warm the caching allocator outside the capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g8, g4 = step()
    for rep in range(4):
        say(f"graph replay {rep}")
        x8.copy_(workloads.activations(m, k, seed=300 + rep, device=DEV))
        x4.copy_(workloads.activations(m4, k4, seed=400 + rep, device=DEV))
        graph.replay()
        e8, e4 = step()  # eager, same inputs
        torch.cuda.synchronize()
        assert torch.equal(g8.view(torch.int16), e8.view(torch.int16)), f"replay {rep}: FP8 output differs"
        assert torch.equal(g4.view(torch.int16), e4.view(torch.int16)), f"replay {rep}: MXFP4 output differs"
        if rep:
            assert not torch.equal(g8, prev), "the replay did not follow its new inputs"
        prev = g8.clone()


def test_two_graphs_replayed_concurrently_on_two_streams():
    # two graphs of the same split-K plan, captured one after the other on one stream, replayed at the same
    # time on two streams: each owns its scratch, so both outputs stay right
    m, n, k = 16, 4096, 16384
    b, bs = workloads.blockwise_fp8_weight(n, k, seed=5, device=DEV)
    bb = layouts.shuffle_weight(b)
    xs = [workloads.activations(m, k, seed=500 + i, device=DEV) for i in range(2)]
    qs = [aklr_amd.per_group_quant_fp8(x) for x in xs]
    want = [aklr_amd.gemm_a8w8_blockwise_scaled(q, bb, s.view(m, k // 128), bs, operand_format="none:preshuffled")
            for q, s in qs]
    graphs, outs = [], []
    for q, s in qs:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs.append(aklr_amd.gemm_a8w8_blockwise_scaled(q, bb, s.view(m, k // 128), bs,
                                                            operand_format="none:preshuffled"))
        graphs.append(g)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rep in range(3):
        say(f"two graphs, round {rep}")
        for st in streams:
            st.wait_stream(torch.cuda.current_stream())
        for g, st in zip(graphs, streams):
            with torch.cuda.stream(st):
                for _ in range(4):
                    g.replay()
        torch.cuda.synchronize()
        for i in range(2):
            assert torch.equal(outs[i].view(torch.int16), want[i].view(torch.int16)), f"graph {i} round {rep}"

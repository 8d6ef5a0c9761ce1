"""The no-allocation FP8 GEMM entry point against the regular one, through the C ABI.

aklr_gemm_a8w8_blockscale_noalloc runs the same kernels and plans as aklr_gemm_a8w8_blockscale with its
split-K scratch in the library's per-GPU device array, so its outputs must equal the regular entry
point's bit for bit: on two calls in a row, the second with a smaller input (the array then holds the
first call's words and partials), on plans that split K (stream and LDS kernels) and one that does not.
(That every plan fits the array is checked on the CPU, in tests/test_abi.py.)
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest
import torch

import aklr_amd
from aklr_amd import _lib, layouts, workloads
from tests.helpers import say

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _inputs(m, n, k, seed):
    x = workloads.activations(m, k, seed=seed, device=DEV)
    q, s = aklr_amd.per_group_quant_fp8(x)  # s: [k/128, m], column-major a_scale
    b, bs = workloads.blockwise_fp8_weight(n, k, seed=seed + 1, device=DEV)
    return q, s, layouts.shuffle_weight(b), bs


def _call(fn, m, n, k, q, s, bb, bs, *ws):
    out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    st = fn(q.data_ptr(), k, bb.data_ptr(), k, s.data_ptr(), 1, m, bs.data_ptr(), bs.stride(0), None, out.data_ptr(),
            n, m, n, k, _lib.FP8_E4M3FN, _lib.B_PRESHUFFLE_16x16, _lib.OUT_BF16, *ws,
            torch.cuda.current_stream().cuda_stream)
    return st, out


# (first call, second smaller call): stream split plans, an LDS split plan after a stream one, and an
# unsplit LDS plan (no scratch) followed by a split stream plan
PAIRS = [((16, 4096, 16384), (4, 2112, 7168)), ((256, 2112, 7168), (128, 2112, 7168)),
         ((2048, 7168, 2048), (64, 2112, 7168))]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_regular_entry(first, second):
    L = _lib.lib()
    for i, (m, n, k) in enumerate((first, second)):
        say(f"noalloc gemm call {i}: m={m} n={n} k={k}")
        need = L.aklr_gemm_a8w8_blockscale_workspace_bytes(m, n, k)
        assert need <= _lib.NOALLOC_SCRATCH_BYTES
        q, s, bb, bs = _inputs(m, n, k, seed=10 * i + m)
        ws = torch.empty(max(need, 16), dtype=torch.uint8, device=DEV)
        st, want = _call(L.aklr_gemm_a8w8_blockscale, m, n, k, q, s, bb, bs, ws.data_ptr(), need)
        assert st == 0, L.aklr_status_string(st)
        st, got = _call(L.aklr_gemm_a8w8_blockscale_noalloc, m, n, k, q, s, bb, bs)
        assert st == 0, L.aklr_status_string(st)
        torch.cuda.synchronize()
        assert not torch.isnan(got.float()).any(), "no-allocation call left outputs unwritten"
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"call {i}: outputs differ"


def _scratch_words() -> np.ndarray:
    """The first 128 KiB (the split-K arrival words) of this device's no-allocation array."""
    L = _lib.lib()
    ptr, nbytes = ctypes.c_void_p(), ctypes.c_size_t()
    assert L.aklr_noalloc_scratch(ctypes.byref(ptr), ctypes.byref(nbytes)) == 0
    assert nbytes.value == _lib.NOALLOC_SCRATCH_BYTES and ptr.value
    words = torch.empty(131072, dtype=torch.uint8, device=DEV)
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hip.hipMemcpy(words.data_ptr(), ptr.value, 131072, 3) == 0  # device to device
    torch.cuda.synchronize()
    return words.cpu().numpy().view(np.uint64)


def test_noalloc_words_idle_after_split_calls():
    """Every split tile's arrival word is reset to the reserved 0 by the workgroup that completes it,
    so after finished calls the array holds no launch tag (the array starts zeroed)."""
    L = _lib.lib()
    for (m, n, k) in ((16, 4096, 16384), (256, 2112, 7168)):
        say(f"noalloc split call then words: m={m} n={n} k={k}")
        q, s, bb, bs = _inputs(m, n, k, seed=77 + m)
        st, _ = _call(L.aklr_gemm_a8w8_blockscale_noalloc, m, n, k, q, s, bb, bs)
        assert st == 0, L.aklr_status_string(st)
        torch.cuda.synchronize()
        w = _scratch_words()
        assert (w == 0).all(), f"{int((w != 0).sum())} arrival words left tagged"


def _graph_check(first_use_in_capture: bool) -> None:
    """Capture aklr_gemm_a8w8_blockscale_noalloc in a torch graph (after an eager warm-up, or as the
    process's first call of it), replay it on new inputs copied into the captured buffers, and compare
    each replay bit for bit with the regular entry point on the same inputs."""
    L = _lib.lib()
    m, n, k = 16, 4096, 16384  # a split-K plan: the array's words and partials are used
    q, s, bb, bs = _inputs(m, n, k, seed=5)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    stream = torch.cuda.Stream()

    def launch():
        st = L.aklr_gemm_a8w8_blockscale_noalloc(q.data_ptr(), k, bb.data_ptr(), k, s.data_ptr(), 1, m,
                                                 bs.data_ptr(), bs.stride(0), None, out.data_ptr(), n, m, n, k,
                                                 _lib.FP8_E4M3FN, _lib.B_PRESHUFFLE_16x16, _lib.OUT_BF16,
                                                 torch.cuda.current_stream().cuda_stream)
        assert st == 0, L.aklr_status_string(st)

    if not first_use_in_capture:
        with torch.cuda.stream(stream):
            launch()
        torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        launch()
    torch.cuda.synchronize()
    need = L.aklr_gemm_a8w8_blockscale_workspace_bytes(m, n, k)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    for rep in range(3):
        q2, s2, bb2, bs2 = _inputs(m, n, k, seed=100 + rep)
        q.copy_(q2), s.copy_(s2), bb.copy_(bb2), bs.copy_(bs2)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        st, want = _call(L.aklr_gemm_a8w8_blockscale, m, n, k, q, s, bb, bs, ws.data_ptr(), need)
        assert st == 0
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"replay {rep} differs"


def test_noalloc_graph_capture_after_warmup():
    say("noalloc graph capture after an eager call")
    _graph_check(first_use_in_capture=False)


_FRESH = textwrap.dedent("""
    import sys
    sys.path.insert(0, {root!r})
    from tests import test_zz_no_alloc as t
    t._graph_check(first_use_in_capture=True)
    print("fresh-process capture ok", flush=True)
""")


def test_noalloc_graph_capture_first_use_fresh_process():
    """The entry point's first call in a process made inside a capture: its once-per-device address
    lookup then happens during the capture."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    say("noalloc graph capture as the first use, in a child process")
    res = subprocess.run([sys.executable, "-c", _FRESH.format(root=root)], capture_output=True, text=True,
                         timeout=110, cwd=root)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-4000:]
    assert "fresh-process capture ok" in res.stdout

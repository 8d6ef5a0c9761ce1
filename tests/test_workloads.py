"""Synthetic-input generators of the benchmark configurations, on the CPU: the torch MXFP4 weight
quantizer equals the oracle's MXFP4 rule, FP8 weights carry s = amax / 448 per 128 x 128 block (the
partial last row block included), routing draws distinct experts with a Zipf skew."""
from __future__ import annotations

import numpy as np
import torch

from aklr_amd import workloads as w
from oracle import formats as f
from oracle import quant as q


def test_mxfp4_weight_quantizer_matches_oracle():
    x = w.activations(37, 1024, seed=3)
    x[0, :32] = 0
    packed, scales = w.mxfp4_quantize(x)
    bits = x.view(torch.int16).numpy().view(np.uint16)
    want_p, want_s = q.dynamic_mxfp4_quant(bits)
    assert np.array_equal(packed.numpy(), want_p) and np.array_equal(scales.numpy(), want_s)


def test_fp8_block_weight():
    codes, s = w.blockwise_fp8_weight(144, 256, seed=1)
    assert codes.shape == (144, 256) and s.shape == (2, 2)
    g = torch.Generator().manual_seed(1)
    wf = torch.randn((144, 256), generator=g) * 0.02
    for nb in range(2):
        for kb in range(2):
            blk = wf[nb * 128:(nb + 1) * 128, kb * 128:(kb + 1) * 128]
            assert s[nb, kb] == blk.abs().amax() / 448.0
            dq = f.fp8_to_f32(codes[nb * 128:(nb + 1) * 128, kb * 128:(kb + 1) * 128].view(torch.uint8).numpy())
            assert np.max(np.abs(dq * s[nb, kb].item() - blk.numpy())) <= s[nb, kb].item() * 16  # half ulp at 448


def test_activations_outliers_and_seed():
    a = w.activations(64, 1024, seed=5)
    assert a.dtype == torch.bfloat16 and torch.equal(a, w.activations(64, 1024, seed=5))
    big = (a.float().abs() > 6).float().mean().item()
    assert 0.003 < big < 0.02  # ~1% of entries x20


def test_zipf_routing():
    ids = w.zipf_routing(4096)
    assert ids.shape == (4096, 8)
    srt = ids.sort(dim=1).values
    assert bool((srt[:, 1:] != srt[:, :-1]).all())
    counts = torch.bincount(ids.reshape(-1), minlength=256)
    assert counts[0] > counts[255] * 10 and int((counts > 0).sum()) == 256

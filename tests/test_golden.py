"""The CPU oracle against the golden fixtures of tests/golden/ (written by make_golden.py from an
independent torch restatement and float64 products, not from the oracle): quantizers bit-exact,
GEMMs within float32 accumulation error of the float64 product."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import gemm as ogemm
from oracle import quant as oquant

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


QUANT = sorted(p.name for p in GOLDEN.glob("quant_*.npz"))
GEMM8 = sorted(p.name for p in GOLDEN.glob("gemm8_*.npz"))
GEMM4 = sorted(p.name for p in GOLDEN.glob("gemm4_*.npz"))


def test_fixtures_present():
    assert len(QUANT) >= 2 and len(GEMM8) >= 3 and len(GEMM4) >= 2


@pytest.mark.parametrize("name", QUANT)
def test_quant_fixtures(name):
    f = _load(name)
    q, s = oquant.per_group_quant_fp8(f["x_bf16_bits"])
    assert np.array_equal(q, f["fp8_codes"])
    assert np.array_equal(s.view(np.uint32), f["fp8_scales"].view(np.uint32))
    q, s = oquant.per_group_quant_mxfp8(f["x_bf16_bits"])
    assert np.array_equal(q, f["mxfp8_codes"]) and np.array_equal(s, f["mxfp8_scales"])
    q, s = oquant.dynamic_mxfp4_quant(f["x_bf16_bits"])
    assert np.array_equal(q, f["mxfp4_packed"]) and np.array_equal(s, f["mxfp4_scales"])


def _close_to_f64(got, want):
    want = np.asarray(want, dtype=np.float64)
    scale = np.sqrt(np.mean(want**2))
    assert np.max(np.abs(got - want)) <= 1e-5 * scale


@pytest.mark.parametrize("name", GEMM8)
def test_gemm8_fixtures(name):
    f = _load(name)
    got = ogemm.gemm_a8w8_blockwise_scaled(f["a"], f["b"], f["a_scale_group_major"], f["b_scale"],
                                           scale_major_mode="MN")
    _close_to_f64(got, f["out_f64"])
    got_k = ogemm.gemm_a8w8_blockwise_scaled(f["a"], f["b"], np.ascontiguousarray(f["a_scale_group_major"].T),
                                             f["b_scale"], scale_major_mode="K")
    assert np.array_equal(got, got_k)


@pytest.mark.parametrize("name", GEMM4)
def test_gemm4_fixtures(name):
    f = _load(name)
    got = ogemm.gemm_a4w4_mxfp4(f["a"], f["b"], f["a_scale"], f["b_scale"])
    _close_to_f64(got, f["out_f64"])

"""The aiter provider without aiter or a GPU: selectors take aiter's exact positional contracts and
decline or offer as the reference's do (tests/plugins/aiter/test_provider_gemm.py of AKLR: the
apis' ``serving`` answers are stood in, aiter's ``plugin`` module is a stand-in)."""
from __future__ import annotations

import sys
import types
from dataclasses import dataclass

import pytest
import torch

from aklr_amd import FallbackReason as FR
from aklr_amd import KernelInfo
from aklr_amd.plugins.aiter import provider as prov
from aklr_amd.plugins.aiter.provider import _base, gemm as pgemm, quant as pquant


@dataclass
class Candidate:
    provider: str
    kernel_id: str
    artifact_digest: str
    qualification: str
    run: object


@pytest.fixture
def aiter(monkeypatch):
    plugin = types.ModuleType("aiter.plugin")
    plugin.KernelCandidate = Candidate
    state = {"enabled": ["other"]}
    plugin.status = lambda: {"enabled": list(state["enabled"])}

    def configure(source, enable):
        state["enabled"] = list(enable)
        state["source"] = source

    plugin.configure = configure
    plugin.state = state
    pkg = types.ModuleType("aiter")
    pkg.plugin = plugin
    monkeypatch.setitem(sys.modules, "aiter", pkg)
    monkeypatch.setitem(sys.modules, "aiter.plugin", plugin)
    monkeypatch.setattr(_base, "_is_ready", True)
    return plugin


class FakeApi:
    """Stands in for an op api: records calls, answers ``serving`` with ``answer``."""

    def __init__(self, answer, result="result"):
        self.answer, self.result, self.calls = answer, result, []

    def serving(self, *args, **kwargs):
        self.calls.append(("serving", args, kwargs))
        return self.answer

    def __call__(self, *args, **kwargs):
        self.calls.append(("call", args, kwargs))
        return self.result


INFO = KernelInfo("gemm_a8w8_blockwise_scaled@1.0", "row_major", "aklr_gemm_a8w8_blockscale:decode", "abc123")


def _op(name):
    return types.SimpleNamespace(name=name)


def _t(shape, dtype=torch.float32):
    return torch.zeros(shape, dtype=dtype)


def test_provider_registration():
    assert set(prov.provider.op_versions) == {"gemm_a8w8_blockscale", "gemm_a8w8_blockscale_bpreshuffle",
                                              "gemm_a8w8_blockscale_out", "per_group_quant"}
    assert prov.provider.name == "aklr" and 1 in prov.provider.api_versions


def test_blockscale_selector(aiter, monkeypatch):
    api = FakeApi(INFO)
    monkeypatch.setattr(pgemm, "gemm_a8w8_blockwise_scaled", api)
    xq, wq, xs, ws = _t((4, 256)), _t((16, 256)), _t((4, 2)), _t((1, 2))
    c = prov.provider.select(_op("gemm_a8w8_blockscale"), (xq, wq, xs, ws, torch.bfloat16, False, None), {})
    assert isinstance(c, Candidate) and c.provider == "aklr" and c.kernel_id == INFO.kernel_ref
    assert c.artifact_digest == "aklr:abc123"
    assert api.calls[-1][2] == {"out_dtype": torch.bfloat16}
    assert c.run(xq, wq, xs, ws, torch.bfloat16, False, None) == "result"
    # declines: preshuffled weight, split_k, non-fp32 scales
    sel = prov.provider.select
    assert sel(_op("gemm_a8w8_blockscale"), (xq, wq, xs, ws, torch.bfloat16, True, None), {}) is None
    assert sel(_op("gemm_a8w8_blockscale"), (xq, wq, xs, ws, torch.bfloat16, False, 2), {}) is None
    assert sel(_op("gemm_a8w8_blockscale"), (xq, wq, xs.half(), ws, torch.bfloat16, False, None), {}) is None
    api.answer = FR.OUT_OF_CONTRACT
    assert sel(_op("gemm_a8w8_blockscale"), (xq, wq, xs, ws, torch.bfloat16, False, None), {}) is None


def test_bpreshuffle_selector_passes_operand_format(aiter, monkeypatch):
    api = FakeApi(INFO)
    monkeypatch.setattr(pgemm, "gemm_a8w8_blockwise_scaled", api)
    xq, wq, xs, ws = _t((4, 256)), _t((16, 256)), _t((4, 2)), _t((1, 2))
    out = _t((4, 16), torch.bfloat16)
    c = prov.provider.select(_op("gemm_a8w8_blockscale_bpreshuffle"), (xq, wq, xs, ws, torch.bfloat16, out), {})
    assert c is not None
    assert api.calls[-1][2] == {"out_dtype": torch.bfloat16, "out": out, "operand_format": "none:preshuffled"}
    xs.is_row_major = True  # aiter reads x_scale column-major: a row-major mark is declined
    assert prov.provider.select(_op("gemm_a8w8_blockscale_bpreshuffle"), (xq, wq, xs, ws, torch.bfloat16, out),
                                {}) is None


def test_blockscale_out_selector(aiter, monkeypatch):
    api = FakeApi(INFO)
    monkeypatch.setattr(pgemm, "gemm_a8w8_blockwise_scaled", api)
    x, w, xs, ws = _t((4, 256)), _t((16, 256)), _t((4, 2)), _t((1, 2))
    y = _t((4, 16), torch.float16)
    args = (x, w, xs, ws, torch.bfloat16, y, None, False, None)
    assert prov.provider.select(_op("gemm_a8w8_blockscale_out"), args, {}) is not None
    # y's dtype wins over dtype, as aiter's Triton GEMM returns y
    assert api.calls[-1][2] == {"out_dtype": torch.float16, "out": y, "operand_format": "none:none"}
    skip = (x, w, xs, ws, torch.bfloat16, y, None, True, None)
    assert prov.provider.select(_op("gemm_a8w8_blockscale_out"), skip, {}) is None
    strided = (x, w, _t((2, 4)).t(), ws, torch.bfloat16, None, None, False, None)
    assert prov.provider.select(_op("gemm_a8w8_blockscale_out"), strided, {}) is None


def test_per_group_quant_selector(aiter, monkeypatch):
    info = KernelInfo("per_group_quant_fp8@1.0", "row_major", "aklr_per_group_quant_fp8", "abc")
    scales = torch.arange(6, dtype=torch.float32).view(2, 3)  # (groups, rows) group-major
    fp8 = FakeApi(info, result=(_t((3, 256)), scales))
    mx = FakeApi(info, result=(_t((3, 256)), torch.zeros((3, 8), dtype=torch.uint8)))
    monkeypatch.setattr(pquant, "per_group_quant_fp8", fp8)
    monkeypatch.setattr(pquant, "per_group_quant_mxfp8", mx)
    x = _t((3, 256), torch.bfloat16)
    e4 = torch.float8_e4m3fn
    args = (x, None, e4, 128, True, None, 1, torch.float32, False)
    c = prov.provider.select(_op("per_group_quant"), args, {})
    q, s = c.run(*args)
    # aiter's (rows, groups) view over the same group-major bytes
    assert s.shape == (3, 2) and torch.equal(s.reshape(-1), scales.reshape(-1))
    mx_args = (x, None, e4, 32, False, None, 1, torch.float8_e8m0fnu, False)
    c = prov.provider.select(_op("per_group_quant"), mx_args, {})
    assert c is not None and c.run(*mx_args)[1].dtype == torch.float8_e8m0fnu
    for bad in ((x, _t(3), e4, 128, True, None, 1, torch.float32, False),
                (x, None, e4, 128, True, 3, 1, torch.float32, False),
                (x, None, e4, 128, True, None, 1, torch.float32, True),
                (x, None, torch.int8, 128, True, None, 1, torch.float32, False),
                (x, None, e4, 128, False, None, 1, torch.float32, False),
                (x, None, e4, 64, True, None, 1, torch.float32, False)):
        assert prov.provider.select(_op("per_group_quant"), bad, {}) is None


def test_served_raises_on_fallback_and_declining(aiter, monkeypatch):
    with pytest.raises(RuntimeError, match="fell back"):
        _base.served(FR.NO_WORKLOAD)
    api = FakeApi(INFO)
    monkeypatch.setattr(pgemm, "gemm_a8w8_blockwise_scaled", api)
    args = (_t((4, 256)), _t((16, 256)), _t((4, 2)), _t((1, 2)), torch.bfloat16, False, None)
    with prov.declining():
        assert prov.provider.select(_op("gemm_a8w8_blockscale"), args, {}) is None
    assert prov.provider.select(_op("gemm_a8w8_blockscale"), args, {}) is not None
    assert prov.provider.select(_op("gemm_a16w16"), args, {}) is None  # not an op served here


def test_not_ready_declines_everything(aiter, monkeypatch):
    monkeypatch.setattr(_base, "_is_ready", False)
    args = (_t((4, 256)), _t((16, 256)), _t((4, 2)), _t((1, 2)), torch.bfloat16, False, None)
    assert prov.provider.select(_op("gemm_a8w8_blockscale"), args, {}) is None


def test_ready_without_gpu_is_false(monkeypatch, native_lib):
    monkeypatch.setattr(_base, "_is_ready", None)
    assert _base.ready() is (torch.cuda.is_available() and "gfx950" in torch.cuda.get_device_properties(0).gcnArchName)


def test_enable_and_plugin_entry_points(aiter, monkeypatch):
    assert prov.enable("test") is True
    assert aiter.state["enabled"] == ["aklr", "other"] and aiter.state["source"] == "test"
    from aklr_amd.plugins import sglang, vllm

    # sglang calls register() with its HookRegistry importable; a stand-in records the start-up hook
    hooks = []
    registry = types.ModuleType("sglang.srt.plugins.hook_registry")
    registry.HookRegistry = types.SimpleNamespace(register=lambda *a: hooks.append(a))
    registry.HookType = types.SimpleNamespace(AROUND="around", AFTER="after")
    for name in ("sglang", "sglang.srt", "sglang.srt.plugins"):
        monkeypatch.setitem(sys.modules, name, types.ModuleType(name))
    monkeypatch.setitem(sys.modules, "sglang.srt.plugins.hook_registry", registry)
    aiter.state["enabled"] = ["other"]
    monkeypatch.setenv("AKLR_AITER_PLUGIN", "1")
    sglang.register()
    assert [h[0] for h in hooks] == [sglang.STARTED_AFTER]
    assert aiter.state["enabled"][0] == "aklr"
    aiter.state["enabled"] = ["other"]
    monkeypatch.setenv("AKLR_DISABLE", "1")
    vllm.register()
    assert aiter.state["enabled"] == ["other"]
    monkeypatch.setenv("AKLR_AITER_PLUGIN", "yes")
    with pytest.raises(SystemExit):
        vllm.register()


def test_enable_without_aiter(monkeypatch):
    monkeypatch.setitem(sys.modules, "aiter", None)
    assert prov.enable() is False

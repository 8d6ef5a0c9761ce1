"""The sglang plugin's route for DeepseekV2MoE.forward_normal, its hook and its switch, on stand-ins of
sglang 0.5.23 (sglang is not installed here): which calls stay on sglang, which arguments the op gets,
and how install() hooks the route (aklr/plugins/sglang/hook.py:29-103,
aklr/plugins/sglang/models/deepseek_v2/api.py:53-151, aklr/plugins/sglang/__init__.py:18-44)."""
from __future__ import annotations

import inspect
import sys
from types import ModuleType, SimpleNamespace

import pytest
import torch

from aklr_amd import FallbackReason as FR
from aklr_amd.plugins.sglang import hook
from aklr_amd.plugins.sglang.models import deepseek_v2 as ds


def _module(monkeypatch, name, **attrs):
    mod = ModuleType(name)
    for k, v in attrs.items():
        setattr(mod, k, v)
    monkeypatch.setitem(sys.modules, name, mod)
    parent, _, child = name.rpartition(".")
    if parent:
        if parent not in sys.modules:
            _module(monkeypatch, parent)
        setattr(sys.modules[parent], child, mod)
    return mod


class _Flag:
    def __init__(self, value=False):
        self.value = value

    def get(self):
        return self.value


def _forward_normal(self, hidden_states, gemm_output_zero_allocator=None, input_ids=None, input_ids_global=None,
                    skip_shared_experts=False, use_vision_topk=False, return_moe_output=False, leave_output_sum=False):
    return "sglang's own forward_normal"


@pytest.fixture
def sglang(monkeypatch):
    """sglang 0.5.23 as far as the route reads it; ``state`` holds the knobs the checks read."""
    state = SimpleNamespace(registered=[], reduced=[], bound=None, a2a_none=True, piecewise=False, breakable=False,
                            use_aiter=True, jit_topk=_Flag(False), uniform=_Flag(False), round_robin=_Flag(False))
    moe = SimpleNamespace(ep_join_mode=None, enable_waterfill=False, enable_eplb=False, init_expert_location="trivial",
                          ep_num_redundant_experts=0, expert_distribution_recorder_mode=None)
    state.exec = SimpleNamespace(moe=moe, deterministic=SimpleNamespace(enable_deterministic_inference=False),
                                 features=SimpleNamespace(enable_return_routed_experts=False))
    state.parallel = SimpleNamespace(dwdp_size=1)
    _module(monkeypatch, "sglang.srt.plugins.hook_registry",
            HookRegistry=SimpleNamespace(register=lambda *a: state.registered.append(a)),
            HookType=SimpleNamespace(AROUND="around", AFTER="after"))
    _module(monkeypatch, "sglang.srt.models.deepseek_v2",
            DeepseekV2MoE=type("DeepseekV2MoE", (), {"forward_normal": _forward_normal}))
    _module(monkeypatch, "sglang.srt.model_executor.forward_context", has_forward_context=lambda: True,
            get_forward_context=lambda: SimpleNamespace(moe_num_token_non_padded=lambda: state.bound))
    _module(monkeypatch, "sglang.srt.environ", envs=SimpleNamespace(
        SGLANG_SIMULATE_UNIFORM_EXPERTS=state.uniform, SGLANG_SIMULATE_ROUND_ROBIN_EXPERTS=state.round_robin,
        SGLANG_OPT_USE_JIT_KERNEL_GROUPED_TOPK=state.jit_topk))
    _module(monkeypatch, "sglang.srt.layers.moe",
            get_moe_a2a_backend=lambda: SimpleNamespace(is_none=lambda: state.a2a_none),
            post_experts_all_reduce=lambda x: state.reduced.append(x) or ("reduced", x))
    topk_mod = _module(monkeypatch, "sglang.srt.layers.moe.topk")
    monkeypatch.setattr(topk_mod, "_use_aiter", True, raising=False)
    state.topk_module = topk_mod
    base = "sglang.srt.model_executor.runner_backend_utils"
    _module(monkeypatch, f"{base}.breakable_cuda_graph.context", is_in_breakable_cuda_graph=lambda: state.breakable)
    _module(monkeypatch, f"{base}.tc_piecewise_cuda_graph.context_manager",
            is_in_tc_piecewise_cuda_graph=lambda: state.piecewise)
    _module(monkeypatch, "sglang.srt.runtime_context", get_exec=lambda: state.exec, get_parallel=lambda: state.parallel)
    monkeypatch.setattr(hook, "sglang_version", lambda: "0.5.23")
    return state


FusedMoE = type("FusedMoE", (), {})
StandardDispatcher = type("StandardDispatcher", (), {})
Fp8MoEMethod = type("Fp8MoEMethod", (), {})
QuarkW4A4MXFp4MoE = type("QuarkW4A4MXFp4MoE", (), {})


def _mlp(grouped=True, reduce_results=False):
    """A DeepseekV2MoE as the route reads it: fp8 experts at 128 x 128 blocks on aiter's fused_moe."""
    config = SimpleNamespace(activation="silu", is_gated=True, apply_router_weight_on_input=False, no_combine=False,
                             gemm1_alpha=None, gemm1_clamp_limit=None, swiglu_limit=None)
    runner = SimpleNamespace(runner_backend=SimpleNamespace(is_aiter=lambda: True), config=config)
    method = Fp8MoEMethod()
    method.block_quant, method.use_mxfp8, method.is_fp4_expert = True, False, False
    method.weight_block_size, method.runner = [128, 128], runner
    experts = FusedMoE()
    experts.quant_method, experts.dispatcher, experts.reduce_results = method, StandardDispatcher(), False
    experts.w13_weight, experts.w2_weight = "w13", "w2"
    experts.w13_weight_scale_inv, experts.w2_weight_scale_inv = "w13_scale_inv", "w2_scale_inv"
    routing = SimpleNamespace(use_grouped_topk=grouped, top_k=9, num_fused_shared_experts=1, num_expert_group=8,
                              topk_group=4, renormalize=True, scoring_func="sigmoid", correction_bias="bias_as_held",
                              correction_bias_for_dtype=lambda dtype: ("bias_in", dtype))
    return SimpleNamespace(experts=experts, topk=SimpleNamespace(topk_config=routing),
                           gate=SimpleNamespace(weight="router_weight", e_score_correction_bias_vl=None),
                           routed_scaling_factor=2.5, reduce_results=reduce_results,
                           _fuse_shared_experts_inside_sbo=False, is_hash=False)


@pytest.fixture
def op(monkeypatch):
    """The op the route calls, recorded."""
    calls = []
    monkeypatch.setattr(ds, "deepseek_v2_fp8_moe", lambda **kw: calls.append(kw) or "op output")
    return calls


def test_route_passes_the_modules_weights_and_routing_to_the_op(sglang, op):
    x = torch.zeros(4, 8, dtype=torch.bfloat16)
    assert ds._moe_forward_normal(_mlp(), x) == "op output"
    (kw,) = op
    assert kw == {"hidden_states": x, "router_weight": "router_weight", "correction_bias": ("bias_in", torch.bfloat16),
                  "w1": "w13", "w1_scale": "w13_scale_inv", "w2": "w2", "w2_scale": "w2_scale_inv", "topk": 8,
                  "num_expert_group": 8, "topk_group": 4, "renormalize": True, "scoring_func": "sigmoid",
                  "routed_scaling_factor": 2.5}


def test_route_ungrouped_top_k_is_one_group_and_takes_the_bias_as_held(sglang, op):
    ds._moe_forward_normal(_mlp(grouped=False), torch.zeros(2, 8))
    assert op[0]["num_expert_group"] == 1 and op[0]["topk_group"] == 1
    assert op[0]["correction_bias"] == "bias_as_held"  # only aiter's grouped top-k reads the dtype copy
    op.clear()
    sglang.jit_topk.value = True  # sglang's JIT grouped top-k reads the bias as held
    ds._moe_forward_normal(_mlp(), torch.zeros(2, 8))
    assert op[0]["correction_bias"] == "bias_as_held"


def test_route_all_reduces_when_the_layer_reduces(sglang, op):
    assert ds._moe_forward_normal(_mlp(reduce_results=True), torch.zeros(2, 8)) == ("reduced", "op output")
    assert sglang.reduced == ["op output"]


def _no_op(monkeypatch):
    monkeypatch.setattr(ds, "deepseek_v2_fp8_moe", lambda **kw: pytest.fail("the op was asked"))


@pytest.mark.parametrize("kwarg", ["skip_shared_experts", "use_vision_topk", "return_moe_output", "leave_output_sum"])
def test_calls_the_op_cannot_take_stay_on_sglang(sglang, monkeypatch, kwarg):
    _no_op(monkeypatch)
    assert ds._moe_forward_normal(_mlp(), torch.zeros(2, 8), **{kwarg: True}) is FR.OUT_OF_CONTRACT


def _set(obj, path, value):
    *head, last = path.split(".")
    for h in head:
        obj = getattr(obj, h)
    setattr(obj, last, value)


@pytest.mark.parametrize("what", [
    "bound", "a2a", "piecewise", "breakable", "ep_join", "dwdp", "deterministic", "waterfill", "eplb", "location",
    "redundant", "recorder", "routed_experts", "uniform", "round_robin"])
def test_runtime_states_keep_the_call_on_sglang(sglang, monkeypatch, what):
    _no_op(monkeypatch)
    setting = {
        "bound": lambda: setattr(sglang, "bound", torch.tensor([3])),
        "a2a": lambda: setattr(sglang, "a2a_none", False),
        "piecewise": lambda: setattr(sglang, "piecewise", True),
        "breakable": lambda: setattr(sglang, "breakable", True),
        "ep_join": lambda: _set(sglang.exec, "moe.ep_join_mode", "join"),
        "dwdp": lambda: _set(sglang.parallel, "dwdp_size", 2),
        "deterministic": lambda: _set(sglang.exec, "deterministic.enable_deterministic_inference", True),
        "waterfill": lambda: _set(sglang.exec, "moe.enable_waterfill", True),
        "eplb": lambda: _set(sglang.exec, "moe.enable_eplb", True),
        "location": lambda: _set(sglang.exec, "moe.init_expert_location", "random"),
        "redundant": lambda: _set(sglang.exec, "moe.ep_num_redundant_experts", 1),
        "recorder": lambda: _set(sglang.exec, "moe.expert_distribution_recorder_mode", "stat"),
        "routed_experts": lambda: _set(sglang.exec, "features.enable_return_routed_experts", True),
        "uniform": lambda: setattr(sglang.uniform, "value", True),
        "round_robin": lambda: setattr(sglang.round_robin, "value", True),
    }[what]
    setting()
    assert ds._moe_forward_normal(_mlp(), torch.zeros(2, 8)) is FR.OUT_OF_CONTRACT


@pytest.mark.parametrize("what", [
    "mxfp4", "not_fused_moe", "dispatcher", "experts_reduce", "not_block", "mxfp8", "fp4_expert", "block_64",
    "no_runner", "not_aiter", "gelu", "not_gated", "weight_on_input", "no_combine", "alpha", "clamp", "swiglu",
    "w13_bias", "fp8_activations", "sbo", "hash", "vl_bias"])
def test_layers_the_op_does_not_take_stay_on_sglang(sglang, monkeypatch, what):
    _no_op(monkeypatch)
    mlp = _mlp()
    ex, method = mlp.experts, mlp.experts.quant_method
    cfg = method.runner.config
    {
        "mxfp4": lambda: setattr(ex, "scheme", QuarkW4A4MXFp4MoE()),
        "not_fused_moe": lambda: setattr(mlp, "experts", SimpleNamespace(**vars(ex))),
        "dispatcher": lambda: setattr(ex, "dispatcher", SimpleNamespace()),
        "experts_reduce": lambda: setattr(ex, "reduce_results", True),
        "not_block": lambda: setattr(method, "block_quant", False),
        "mxfp8": lambda: setattr(method, "use_mxfp8", True),
        "fp4_expert": lambda: setattr(method, "is_fp4_expert", True),
        "block_64": lambda: setattr(method, "weight_block_size", [64, 64]),
        "no_runner": lambda: setattr(method, "runner", None),
        "not_aiter": lambda: setattr(method.runner, "runner_backend", SimpleNamespace(is_aiter=lambda: False)),
        "gelu": lambda: setattr(cfg, "activation", "gelu"),
        "not_gated": lambda: setattr(cfg, "is_gated", False),
        "weight_on_input": lambda: setattr(cfg, "apply_router_weight_on_input", True),
        "no_combine": lambda: setattr(cfg, "no_combine", True),
        "alpha": lambda: setattr(cfg, "gemm1_alpha", 1.702),
        "clamp": lambda: setattr(cfg, "gemm1_clamp_limit", 7.0),
        "swiglu": lambda: setattr(cfg, "swiglu_limit", 7.0),
        "w13_bias": lambda: setattr(ex, "w13_weight_bias", "bias"),
        "fp8_activations": lambda: setattr(ex, "fp8_activations", True),
        "sbo": lambda: setattr(mlp, "_fuse_shared_experts_inside_sbo", True),
        "hash": lambda: setattr(mlp, "is_hash", True),
        "vl_bias": lambda: setattr(mlp.gate, "e_score_correction_bias_vl", "vl"),
    }[what]()
    assert ds._moe_forward_normal(mlp, torch.zeros(2, 8)) is FR.OUT_OF_CONTRACT


def test_a_swiglu_limit_of_zero_is_no_limit(sglang, op):
    mlp = _mlp()
    mlp.experts.quant_method.runner.config.swiglu_limit = 0.0
    assert ds._moe_forward_normal(mlp, torch.zeros(2, 8)) == "op output"


def test_route_takes_its_targets_parameters(sglang):
    target = hook.resolve(ds.TARGET)
    params = lambda f: [(p.name, p.kind, p.default) for p in inspect.signature(f).parameters.values()]
    assert params(ds._moe_forward_normal) == params(target)


def test_the_real_op_declines_cpu_tensors_and_the_hook_runs_sglangs_code(sglang):
    # the real deepseek_v2_fp8_moe on CPU tensors returns OUT_OF_CONTRACT, so the AROUND hook hands the call
    # (same arguments) to sglang's own forward_normal
    route = next(r for r in hook.routes() if r.target == ds.TARGET)
    mlp = _mlp()
    mlp.experts.w13_weight = torch.zeros((17, 256, 256), dtype=torch.float8_e4m3fn)
    mlp.experts.w2_weight = torch.zeros((17, 256, 128), dtype=torch.float8_e4m3fn)
    mlp.experts.w13_weight_scale_inv = torch.ones((17, 2, 2))
    mlp.experts.w2_weight_scale_inv = torch.ones((17, 2, 1))
    mlp.gate.weight = torch.zeros((16, 256), dtype=torch.bfloat16)
    mlp.topk.topk_config.correction_bias_for_dtype = lambda dtype: torch.zeros(16, dtype=dtype)
    seen = []
    orig = lambda *a, **k: seen.append((a, k)) or "sglang's result"
    out = hook.around(route)(orig, mlp, torch.zeros((4, 256), dtype=torch.bfloat16), leave_output_sum=False)
    assert out == "sglang's result" and seen[0][0][0] is mlp and seen[0][1] == {"leave_output_sum": False}


def _route(target, versions=("0.5.23",), eager=False, fn=None):
    return hook.Route(target, versions, fn or (lambda *a, **k: "route"), eager)


def test_install_hooks_the_targets_tested_on_the_installed_sglang(sglang, monkeypatch):
    monkeypatch.setattr(hook, "_ROUTES", [_route(ds.TARGET), _route(ds.TARGET + "_other", versions=("0.5.22",))])
    hook.install()
    assert [(t, kind) for t, _, kind in sglang.registered] == [(ds.TARGET, "around")]


def test_install_skips_a_target_whose_dependency_is_absent_and_stops_on_a_moved_one(sglang, monkeypatch, tmp_path):
    host = tmp_path / "aklr_host_pkg"
    host.mkdir()
    (host / "__init__.py").write_text("")
    (host / "layer.py").write_text("import aklr_absent_dependency\n")
    (host / "kept.py").write_text("class Layer:\n    def forward(self):\n        pass\n")
    monkeypatch.syspath_prepend(str(tmp_path))
    for name in ("aklr_host_pkg", "aklr_host_pkg.layer", "aklr_host_pkg.kept"):
        monkeypatch.delitem(sys.modules, name, raising=False)
    monkeypatch.setattr(hook, "_ROUTES", [_route("aklr_host_pkg.layer.Layer.forward"),
                                          _route("aklr_absent_package.ops.fused_moe"),
                                          _route("aklr_host_pkg.kept.Layer.forward")])
    hook.install()
    assert [t for t, _, _ in sglang.registered] == ["aklr_host_pkg.kept.Layer.forward"]
    for moved in ("aklr_host_pkg.kept.Layer.forward_normal", "aklr_host_pkg.renamed.Layer.forward"):
        monkeypatch.setattr(hook, "_ROUTES", [_route(moved)])
        with pytest.raises(AttributeError):
            hook.install()


def test_resolve_names_modules_classes_and_methods():
    assert hook.resolve("os.path.join") is __import__("os").path.join
    assert hook.resolve("aklr_amd.plugins.sglang.hook.Route") is hook.Route
    with pytest.raises(ModuleNotFoundError):
        hook.resolve("aklr_absent_package.x")


def test_around_falls_back_served_and_compiled(monkeypatch):
    orig = lambda *a, **k: ("orig", a, k)
    served = hook.around(_route("t", fn=lambda *a, **k: ("route", a, k)))
    declines = hook.around(_route("t", fn=lambda *a, **k: FR.OUT_OF_CONTRACT))
    assert served(orig, 1, x=2) == ("route", (1,), {"x": 2})
    assert declines(orig, 1, x=2) == ("orig", (1,), {"x": 2})
    monkeypatch.setattr(torch.compiler, "is_compiling", lambda: True)
    assert served(orig, 1) == ("orig", (1,), {})  # under Dynamo a plain route leaves the call to sglang
    eager = hook.around(_route("t", eager=True, fn=lambda *a, **k: "route"))
    assert eager(orig, 1) == "route"


def test_sglang_version_drops_only_a_local_label(monkeypatch):
    monkeypatch.undo()
    monkeypatch.setattr(hook, "version", lambda dist: "0.5.23+rocm7.0")
    assert hook.sglang_version() == "0.5.23"
    monkeypatch.setattr(hook, "version", lambda dist: "0.5.23.dev20261201+g5bebe7a")
    assert hook.sglang_version() == "0.5.23.dev20261201"


@pytest.mark.parametrize("env,installs", [({}, False), ({"AKLR_SGLANG_PLUGIN": "1"}, True),
                                          ({"AKLR_SGLANG_PLUGIN": "1", "AKLR_DISABLE": "1"}, False),
                                          ({"AKLR_SGLANG_PLUGIN": "0"}, False)])
def test_register_switch(sglang, monkeypatch, env, installs):
    import aklr_amd.plugins.sglang as plugin

    for k, v in env.items():
        monkeypatch.setenv(k, v)
    installed = []
    monkeypatch.setattr(hook, "install", lambda: installed.append(True))
    plugin.register()
    assert installed == ([True] if installs else [])
    # the library starts after sglang's torch.distributed set-up, whatever the switches say
    assert (plugin.STARTED_AFTER, plugin._start_library, "after") in sglang.registered


def test_register_ends_the_process_on_a_bad_switch(sglang, monkeypatch):
    import aklr_amd.plugins.sglang as plugin

    monkeypatch.setenv("AKLR_SGLANG_PLUGIN", "yes")
    with pytest.raises(SystemExit, match="AKLR_SGLANG_PLUGIN"):
        plugin.register()

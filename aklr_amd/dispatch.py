"""Dispatch semantics of the op APIs (the drop-in boundary's contract).

Mirrors aklr/core/runtime/dispatch/_dispatcher.py:
- an api call returns its outputs, or a ``FallbackReason`` when this library does not serve the call
  (the caller then runs its own code); it never raises for a call it does not serve
  (_dispatcher.py:53-70, :192-240);
- ``api.serving(...)`` answers the same question without running anything: the ``KernelInfo`` of the
  kernel that would serve the call, or the reason (:248-263); ``api.fallback_reason(...)`` is ``None``
  or the reason (:242-246);
- ``AKLR_DISABLE``: ``"1"`` closes every op, ``"0"`` or unset none, anything else is a
  comma-separated list of contract ids (``per_group_quant_fp8@1.0``) to close; a closed op returns
  ``FallbackReason.DISABLED`` (aklr/core/platform/env.py:59-64);
- ``AKLR_TRACE``: ``"0"``/unset, ``"plugin"``, ``"op"`` or ``"all"`` (any other value raises
  ``ValueError``, env.py:44-50); ``op``/``all`` log each distinct (op, variant, outcome) once per
  process (aklr/core/runtime/dispatch/_trace.py:36-100).

What differs by design: there is no per-shape dispatch table. Every in-contract call that reaches a
supported layout is served by the compiled HIP kernels; nothing compiles at call time, so a call first
met inside a graph capture is served too (its split-K scratch is a per-call ``torch.empty``, which a
capture takes from the graph's pool; ``aklr_amd.workspace``). Layouts the kernels do not implement
return ``NO_WORKLOAD``. A kernel that fails raises; it does not fall back (_dispatcher.py:217-229).
"""
from __future__ import annotations

import enum
import logging
import os
import threading
from dataclasses import dataclass

_LOGGER = logging.getLogger("aklr_amd")


class FallbackReason(str, enum.Enum):
    """Why an api call did not run an aklr_amd kernel; the caller then runs its own."""

    NO_SCHEMA = "no_schema"
    DISABLED = "disabled"
    OUT_OF_CONTRACT = "out_of_contract"
    NO_WORKLOAD = "no_workload"
    NOT_MEASURED = "not_measured"
    INACCURATE = "inaccurate"
    NOT_QUALIFIED = "not_qualified"
    NOT_WARMED = "not_warmed"


@dataclass(frozen=True)
class KernelInfo:
    """What ``serving`` returns for a served call (the role of the reference's RunnableMetadata)."""

    contract_id: str
    variant: str
    kernel_ref: str  # "<library symbol>:<path>" e.g. "aklr_gemm_a8w8_blockscale:decode"
    content_hash: str  # sha256 prefix of the loaded library
    build_type: str = "hip"


ENV_DISABLE = "AKLR_DISABLE"
ENV_TRACE = "AKLR_TRACE"
ENV_AITER_PLUGIN = "AKLR_AITER_PLUGIN"
ENV_SGLANG_PLUGIN = "AKLR_SGLANG_PLUGIN"


def all_disabled() -> bool:
    return (os.environ.get(ENV_DISABLE) or "0") == "1"


def disabled(contract_id: str) -> bool:
    value = os.environ.get(ENV_DISABLE) or "0"
    if value == "1":
        return True
    if value == "0":
        return False
    return contract_id in {item.strip() for item in value.split(",")}


def trace_mode() -> str:
    mode = os.environ.get(ENV_TRACE) or "0"
    if mode not in ("0", "plugin", "op", "all"):
        raise ValueError(f"{ENV_TRACE}={mode!r}: expected '0', 'plugin', 'op' or 'all'")
    return mode


def aiter_plugin_enabled() -> bool:
    value = os.environ.get(ENV_AITER_PLUGIN) or "0"
    if value not in ("0", "1"):
        raise ValueError(f"{ENV_AITER_PLUGIN}={value!r}: expected '1' or '0'")
    return value == "1"


def sglang_plugin_enabled() -> bool:
    """``AKLR_SGLANG_PLUGIN``: "1" hooks sglang's layers to this library's ops, "0" or unset does not;
    any other value raises (aklr/core/platform/env.py:68-72)."""
    value = os.environ.get(ENV_SGLANG_PLUGIN) or "0"
    if value not in ("0", "1"):
        raise ValueError(f"{ENV_SGLANG_PLUGIN}={value!r}: expected '1' or '0'")
    return value == "1"


_trace_seen: set = set()
_trace_lock = threading.Lock()


def plugin_trace(host: str, target: str, route: str, fallback) -> None:
    """With ``AKLR_TRACE`` at "plugin" or "all": log once per (host, target, route, outcome) whether a
    hooked host function ran this library's route or went back to the host's own code."""
    if trace_mode() not in ("plugin", "all"):
        return
    key = ("plugin", host, target, route, str(fallback))
    with _trace_lock:
        if key in _trace_seen:
            return
        _trace_seen.add(key)
    if fallback is None:
        _LOGGER.info("aklr_amd: %s %s served by %s", host, target, route)
    else:
        _LOGGER.info("aklr_amd: %s %s back to %s: %s", host, target, host, fallback.value)


def trace(contract_id: str, variant: str | None, outcome) -> None:
    if trace_mode() not in ("op", "all"):
        return
    key = (contract_id, variant, str(outcome))
    with _trace_lock:
        if key in _trace_seen:
            return
        _trace_seen.add(key)
    if isinstance(outcome, FallbackReason):
        _LOGGER.info("aklr_amd: %s [%s] fallback: %s", contract_id, variant, outcome.value)
    else:
        _LOGGER.info("aklr_amd: %s [%s] served by %s", contract_id, variant, outcome)


# ---------------------------------------------------------------------------------------------
# in-contract helpers shared by the ops (aklr/core/contract/fastkey/_fast_key_fn.py:40, :239-303)
ALIGN = 16


def aligned(t) -> bool:
    return t.data_ptr() % ALIGN == 0


def overlaps(a, b) -> bool:
    """Whether two tensors' storage byte ranges intersect."""
    if a is None or b is None or a.numel() == 0 or b.numel() == 0:
        return False
    a0 = a.data_ptr()
    b0 = b.data_ptr()
    a1 = a0 + _extent_bytes(a)
    b1 = b0 + _extent_bytes(b)
    return a0 < b1 and b0 < a1


def _extent_bytes(t) -> int:
    span = 1 + sum((s - 1) * abs(st) for s, st in zip(t.shape, t.stride()))
    return span * t.element_size()


def on_gpu(*tensors) -> bool:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            return False
        if dev is None:
            dev = t.device
        elif t.device != dev:
            return False
    return True


def api(contract_id: str, run_fn):
    """Decorator binding an op. The decorated function has the op's exact signature and returns a
    plan object (with ``.variant`` and ``.kernel_ref``) or a FallbackReason; ``run_fn(plan)``
    launches and returns the outputs. The result is the api function, with ``.serving`` and
    ``.fallback_reason`` of the same signature attached."""
    import functools

    from . import _lib

    def bind(plan_fn):
        def _plan(*args, **kwargs):
            trace_mode()  # a bad AKLR_TRACE raises on every call, as the reference's RuntimeEnv() does
            if disabled(contract_id):
                return FallbackReason.DISABLED
            return plan_fn(*args, **kwargs)

        @functools.wraps(plan_fn)
        def serving(*args, **kwargs):
            plan = _plan(*args, **kwargs)
            if isinstance(plan, FallbackReason):
                trace(contract_id, None, plan)
                return plan
            return KernelInfo(contract_id, plan.variant, plan.kernel_ref, _lib.digest())

        @functools.wraps(plan_fn)
        def fallback_reason(*args, **kwargs):
            served = serving(*args, **kwargs)
            return served if isinstance(served, FallbackReason) else None

        @functools.wraps(plan_fn)
        def call(*args, **kwargs):
            plan = _plan(*args, **kwargs)
            if isinstance(plan, FallbackReason):
                trace(contract_id, None, plan)
                return plan
            result = run_fn(plan)
            trace(contract_id, plan.variant, plan.kernel_ref)
            return result

        call.serving = serving
        call.fallback_reason = fallback_reason
        call.contract_id = contract_id
        return call

    return bind

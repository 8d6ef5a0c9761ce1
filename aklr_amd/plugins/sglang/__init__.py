"""sglang plugin entry point (``sglang.srt.plugins``; aklr/plugins/sglang/__init__.py:18-44).

- The native library starts right after sglang sets up torch.distributed (an AFTER hook on
  ``ModelRunner.init_torch_distributed``, where the reference starts its dispatcher): a missing or
  stale library then ends the start-up instead of the first forward.
- ``AKLR_AITER_PLUGIN=1`` enables the aiter provider, so sglang's fp8 block-quant linears and group
  quantization reach this library through aiter's routed ops.
- ``AKLR_SGLANG_PLUGIN=1`` hooks sglang's layers to this library's ops through the routes declared in
  ``aklr_amd.plugins.sglang.models`` (the DeepSeek-V2/V3 MoE's forward_normal).
- ``AKLR_DISABLE=1`` leaves both off. A plugin that cannot start ends the process, which sglang would
  only log.
"""
from __future__ import annotations

import importlib

from ...dispatch import aiter_plugin_enabled, all_disabled, sglang_plugin_enabled
from . import hook

__all__ = ["register", "STARTED_AFTER"]

STARTED_AFTER = "sglang.srt.model_executor.model_runner.ModelRunner.init_torch_distributed"
ROUTE_MODULES = (f"{__name__}.models.deepseek_v2",)


def register() -> None:
    """Entry point sglang calls once per process."""
    try:
        _register()
    except Exception as e:
        raise SystemExit(f"aklr_amd: the sglang plugin cannot start: {e!r}") from e


def _start_library(result, *args, **kwargs):
    from ... import _lib

    _lib.lib()
    return result


def _register() -> None:
    from sglang.srt.plugins.hook_registry import HookRegistry, HookType

    HookRegistry.register(STARTED_AFTER, _start_library, HookType.AFTER)
    if aiter_plugin_enabled() and not all_disabled():
        from ..aiter.provider import enable

        enable("aklr_amd sglang plugin, AKLR_AITER_PLUGIN=1")
    if all_disabled() or not sglang_plugin_enabled():
        return
    for module in ROUTE_MODULES:
        importlib.import_module(module)  # declares the module's routes
    hook.install()

"""vLLM plugin entry point (``vllm.general_plugins``; aklr/plugins/vllm/__init__.py:20-61).

vLLM reaches the fp8 block path only through aiter's routed ops (aklr/plugins/README.md:42-48), so
this registers the aiter provider under ``AKLR_AITER_PLUGIN=1`` (and not ``AKLR_DISABLE=1``) and
nothing else. A plugin that cannot start ends the process.
"""
from __future__ import annotations

from ...dispatch import aiter_plugin_enabled, all_disabled

__all__ = ["register"]


def register() -> None:
    try:
        if aiter_plugin_enabled() and not all_disabled():
            from ..aiter.provider import enable

            enable("aklr_amd vllm plugin, AKLR_AITER_PLUGIN=1")
    except Exception as e:
        raise SystemExit(f"aklr_amd: the vllm plugin cannot start: {e!r}") from e

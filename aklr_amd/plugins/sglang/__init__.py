"""sglang plugin entry point (``sglang.srt.plugins``; aklr/plugins/sglang/__init__.py:18-44).

Only the aiter provider is wired here: with ``AKLR_AITER_PLUGIN=1`` (and not ``AKLR_DISABLE=1``) the
provider is enabled, so sglang's fp8 block-quant linears and group quantization reach this library
through aiter's routed ops. A plugin that cannot start ends the process, which sglang would only log.
"""
from __future__ import annotations

from ...dispatch import aiter_plugin_enabled, all_disabled

__all__ = ["register"]


def register() -> None:
    try:
        if aiter_plugin_enabled() and not all_disabled():
            from ..aiter.provider import enable

            enable("aklr_amd sglang plugin, AKLR_AITER_PLUGIN=1")
    except Exception as e:
        raise SystemExit(f"aklr_amd: the sglang plugin cannot start: {e!r}") from e

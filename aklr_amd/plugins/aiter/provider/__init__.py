# SPDX-License-Identifier: MIT
# Copyright (C) 2026, Advanced Micro Devices, Inc. All rights reserved.
# The host protocol and rules here follow aklr/plugins/aiter/provider/__init__.py, whose licence notice this is.

"""aklr_amd as a kernel plugin of aiter (``aiter.plugin``; aklr/plugins/aiter/provider/__init__.py).

Before each call of an op aiter routes, aiter asks its enabled providers whether they serve it.
``Provider.select`` answers from the op apis' ``serving`` (nothing runs) and declines whatever this
library does not serve, so aiter runs its own kernel. aiter finds ``provider`` through the
``aiter.plugins`` entry point and asks it once it is enabled: ``enable()`` does that, called by the
sglang and vLLM plugins under ``AKLR_AITER_PLUGIN=1`` or by any other host.

Served ops: ``gemm_a8w8_blockscale``, ``gemm_a8w8_blockscale_bpreshuffle``,
``gemm_a8w8_blockscale_out`` (module ``gemm``) and ``per_group_quant`` (module ``quant``).
"""
from __future__ import annotations

import logging
from collections.abc import Mapping
from typing import Any

from . import gemm as _gemm  # noqa: F401  (registers its selectors)
from . import quant as _quant  # noqa: F401
from ._base import NAME, SELECTORS, declining, is_declining, ready

__all__ = ["NAME", "Provider", "declining", "enable", "provider"]

_LOGGER = logging.getLogger("aklr_amd.plugins.aiter")


class Provider:
    """The provider aiter asks: ``select`` per call of an op in ``op_versions``."""

    name = NAME
    api_versions = frozenset({1})
    op_versions = {op: frozenset({version}) for op, (version, _) in SELECTORS.items()}

    def select(self, op: Any, args: tuple, kwargs: Mapping[str, Any]) -> Any:
        entry = SELECTORS.get(op.name)
        if entry is None or is_declining() or not ready():
            return None
        return entry[1](args, kwargs)


provider = Provider()


def enable(source: str = "aklr_amd") -> bool:
    """Have aiter ask this provider first, keeping the providers already enabled after it; False when
    the installed aiter has no plugin interface."""
    try:
        from aiter import plugin
    except ImportError:
        _LOGGER.info("aklr_amd: this aiter has no plugin interface (aiter.plugin); its ops stay aiter's")
        return False
    enabled = [name for name in plugin.status()["enabled"] if name != NAME]
    plugin.configure(source=source, enable=[NAME, *enabled])
    return True

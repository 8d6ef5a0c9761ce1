# SPDX-License-Identifier: MIT
# Copyright (C) 2026, Advanced Micro Devices, Inc. All rights reserved.
# The host protocol and rules here follow aklr/plugins/aiter/provider/_base.py, whose licence notice this is.

"""What every selector of the aiter provider shares (aklr/plugins/aiter/provider/_base.py:1-97).

- ``selector(op)`` registers the function that answers aiter's ``op``: it takes the call as aiter
  hands it (positional args with defaults applied, then keyword-only ones) and returns ``offer(...)``'s
  candidate or ``None`` (decline: aiter runs its own kernel).
- ``ready()`` starts this library once per process: the HIP library loads and a gfx950 device is
  visible. A process where that fails declines every call instead of failing aiter's.
- ``offer(serving, run)`` wraps an api's ``serving`` answer in aiter's ``KernelCandidate``.
- ``served(result)`` is the api's result inside ``run``; a fallback there is a bug and raises,
  because aiter does not fall back once ``run`` started.
- ``declining()`` makes this thread decline every call inside the block.
"""
from __future__ import annotations

import contextlib
import logging
import threading
from collections.abc import Callable, Iterator, Mapping
from typing import Any

from ....dispatch import FallbackReason

NAME = "aklr"
QUALIFICATION = "aklr_amd: gfx950 HIP kernels, parity-checked against the AKLR reference formulas"
_LOGGER = logging.getLogger("aklr_amd.plugins.aiter")

Selector = Callable[[tuple, Mapping[str, Any]], Any]
# aiter op name -> (contract version served, selector)
SELECTORS: dict[str, tuple[int, Selector]] = {}
_is_ready: bool | None = None
_ready_lock = threading.Lock()
_declining = threading.local()


def selector(op: str, version: int = 1) -> Callable[[Selector], Selector]:
    def register(fn: Selector) -> Selector:
        if op in SELECTORS:
            raise ValueError(f"aiter op {op!r} already has a selector")
        SELECTORS[op] = (version, fn)
        return fn

    return register


def _start() -> None:
    """Load the native library and check the device is gfx950 (the kernels' only target)."""
    import torch

    from .... import _lib

    _lib.lib()
    if not torch.cuda.is_available():
        raise RuntimeError("no GPU visible")
    arch = getattr(torch.cuda.get_device_properties(torch.cuda.current_device()), "gcnArchName", "")
    if not arch.startswith("gfx950"):
        raise RuntimeError(f"device {arch!r} is not gfx950")


def ready() -> bool:
    global _is_ready
    if _is_ready is None:
        with _ready_lock:
            if _is_ready is None:
                try:
                    _start()
                    _is_ready = True
                except Exception as e:  # noqa: BLE001 (this library's failure must not fail aiter's call)
                    _LOGGER.warning("aklr_amd: serves no aiter op in this process: %r", e)
                    _is_ready = False
    return _is_ready


def reset_ready() -> None:
    """Forget the start-up outcome (tests)."""
    global _is_ready
    _is_ready = None


def offer(serving, run: Callable[..., Any]) -> Any:
    if isinstance(serving, FallbackReason):
        return None
    from aiter import plugin

    return plugin.KernelCandidate(
        provider=NAME,
        kernel_id=serving.kernel_ref,
        artifact_digest=f"aklr:{serving.content_hash}",
        qualification=QUALIFICATION,
        run=run,
    )


def served(result: Any) -> Any:
    if isinstance(result, FallbackReason):
        raise RuntimeError(f"aklr_amd: an accepted aiter call fell back ({result.value})")
    return result


@contextlib.contextmanager
def declining() -> Iterator[None]:
    previous = getattr(_declining, "active", False)
    _declining.active = True
    try:
        yield
    finally:
        _declining.active = previous


def is_declining() -> bool:
    return getattr(_declining, "active", False)

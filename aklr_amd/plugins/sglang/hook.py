# SPDX-License-Identifier: MIT
# Copyright (C) 2025-2026, Advanced Micro Devices, Inc. All rights reserved.
# The host protocol and rules here follow aklr/plugins/sglang/hook.py, whose licence notice this is.

"""How a sglang function reaches this library's ops: a route declared next to the op it calls.

Same protocol as aklr/plugins/sglang/hook.py:29-103:
- ``@sglang_route(target, versions=...)`` declares that the sglang function ``target`` (a dotted path,
  e.g. a method) runs through the decorated route on the sglang releases ``versions`` it was tested on;
- ``install()`` wraps each declared target that the installed sglang release is listed for into sglang's
  ``HookRegistry`` as an AROUND hook. A target whose module needs a package this environment lacks is
  skipped (such a target is never called); a target missing from an installed package is a renamed
  one, which stops the start-up;
- at call time the route runs the op; a route that returns a ``FallbackReason`` hands the call to
  sglang's own code, with the same arguments. Where Dynamo compiles the caller, the call goes to
  sglang, unless the route was declared ``eager``: it then runs outside the compiled graph.
"""
from __future__ import annotations

import importlib
import importlib.util
import logging
from dataclasses import dataclass
from importlib.metadata import version
from typing import Callable

import torch

from ...dispatch import FallbackReason, plugin_trace

__all__ = ["install", "resolve", "sglang_route", "sglang_version", "routes"]

_LOGGER = logging.getLogger("aklr_amd")


@dataclass(frozen=True)
class Route:
    target: str
    versions: tuple[str, ...]
    fn: Callable
    eager: bool


_ROUTES: list[Route] = []


def routes() -> list[Route]:
    return list(_ROUTES)


def sglang_route(target: str, *, versions: tuple[str, ...], eager: bool = False) -> Callable[[Callable], Callable]:
    """Declare ``target``'s route (the decorated function takes ``target``'s parameters)."""

    def declare(fn: Callable) -> Callable:
        _ROUTES.append(Route(target, tuple(versions), fn, eager))
        return fn

    return declare


def sglang_version() -> str:
    """The installed sglang release without its local label: 0.5.23+rocm7.0 is 0.5.23."""
    from packaging.version import Version

    return Version(version("sglang")).public


def resolve(target: str):
    """The object a dotted path names: its longest importable module prefix, then attributes. Unlike
    ``pkgutil.resolve_name``, an import that fails inside a module of the path raises as it is, so a
    module whose dependency is missing is told apart from a path that names no module."""
    parts = target.split(".")
    modname = parts.pop(0)
    obj = importlib.import_module(modname)
    while parts:
        name = f"{modname}.{parts[0]}"
        try:
            obj = importlib.import_module(name)
        except ModuleNotFoundError as e:
            if e.name != name:
                raise  # the module exists and imports a package that is missing
            break
        modname = name
        parts.pop(0)
    for p in parts:
        obj = getattr(obj, p)
    return obj


def install() -> None:
    """Hook every declared target that the installed sglang release was tested for."""
    from sglang.srt.plugins.hook_registry import HookRegistry, HookType

    installed = sglang_version()
    hooked, untested, absent = 0, [], []
    for route in _ROUTES:
        if installed not in route.versions:
            untested.append(route.target)
            continue
        try:
            resolve(route.target)
        except ModuleNotFoundError as e:
            package = (e.name or "").partition(".")[0]
            if not package or importlib.util.find_spec(package) is not None:
                raise  # the target moved within an installed package: the route is stale
            absent.append(f"{route.target} ({package} is not installed)")
            continue
        HookRegistry.register(route.target, around(route), HookType.AROUND)
        hooked += 1
    _LOGGER.warning("aklr_amd hooks %d sglang functions on sglang %s%s%s", hooked, installed,
                    f"; not {', '.join(untested)}, untested on it" if untested else "",
                    f"; not {', '.join(absent)}" if absent else "")


def around(route: Route) -> Callable:
    """The AROUND hook of ``route``: ``hook(orig, *args, **kwargs)``."""
    name = f"{route.fn.__module__}.{route.fn.__qualname__}"

    def serve(orig, args, kwargs):
        result = route.fn(*args, **kwargs)
        fallback = result if isinstance(result, FallbackReason) else None
        plugin_trace("sglang", route.target, name, fallback)
        return orig(*args, **kwargs) if fallback is not None else result

    serve_eagerly = torch.compiler.disable(serve) if route.eager else None

    def hook(orig, *args, **kwargs):
        if not torch.compiler.is_compiling():
            return serve(orig, args, kwargs)
        if serve_eagerly is not None:
            return serve_eagerly(orig, args, kwargs)
        return orig(*args, **kwargs)

    return hook

"""Split-K workspaces for the GEMM entry points.

The C ABI takes a caller-provided workspace whose leading split-K arrival counters must be zero before
first use; every call leaves them zero again. This module keeps one such buffer per (device, stream):
zero-filled when created, grown by doubling, and reused by every later call on that stream. Calls on
one stream are ordered, so they may share it; another stream gets its own buffer.

A buffer that a HIP graph may have captured is never freed. A grown-out buffer is retired, not
released, so an older graph that holds its address stays valid. A call first met inside a graph
capture, whose workspace would need allocating there, is not served (``FallbackReason.NOT_WARMED``,
as aklr/core/runtime/dispatch/_dispatcher.py:164-165): warm each shape eagerly before capturing it.
"""
from __future__ import annotations

import threading

import torch

_lock = threading.Lock()
_buffers: dict[tuple[int, int], torch.Tensor] = {}
_retired: list[torch.Tensor] = []


def _key(device: torch.device) -> tuple[int, int]:
    return device.index if device.index is not None else torch.cuda.current_device(), \
        torch.cuda.current_stream(device).cuda_stream


def capturing(device: torch.device) -> bool:
    return device.type == "cuda" and torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def ready(device: torch.device, nbytes: int) -> bool:
    """Whether a call needing ``nbytes`` can run now without allocating during a graph capture."""
    if nbytes == 0 or not capturing(device):
        return True
    buf = _buffers.get(_key(device))
    return buf is not None and buf.numel() >= nbytes


def get(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """A zero-countered workspace of at least ``nbytes`` for the current stream of ``device``."""
    if nbytes == 0:
        return None
    key = _key(device)
    with _lock:
        buf = _buffers.get(key)
        if buf is None or buf.numel() < nbytes:
            size = max(nbytes, 2 * buf.numel() if buf is not None else 0, 1 << 20)
            if buf is not None:
                _retired.append(buf)
            buf = torch.zeros(size, dtype=torch.uint8, device=device)
            _buffers[key] = buf
    return buf

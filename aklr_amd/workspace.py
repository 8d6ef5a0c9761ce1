"""Split-K workspaces for the GEMM entry points.

The reference's kernel rule (aklr/ops/README.md:214, :276-286) is that scratch is allocated inside the
call, on an argument's device, and that no call depends on what an earlier one left. The C ABI keeps it:
its split-K arrival words carry a tag of the launch (the HSA dispatch id and queue), so a workspace with
any content serves. Each call therefore takes a fresh ``torch.empty`` buffer from torch's caching
allocator on the current stream. Inside a CUDA-graph capture that allocation comes from the graph's
private pool, so every captured graph owns its scratch and two graphs replayed at once on two streams
never share it.
"""
from __future__ import annotations

import torch


def get(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """A scratch buffer of ``nbytes`` (16-byte aligned, contents arbitrary) for one call, or None."""
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)

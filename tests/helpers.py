"""Shared test helpers: tensor <-> numpy views and the oracle checks used by several GPU tests."""
from __future__ import annotations

import sys

import numpy as np
import torch


def say(msg: str) -> None:
    """Name the case before each GPU step (flushed), so a run that ends early still names it."""
    print(msg, flush=True)
    sys.stdout.flush()


def u8(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    return (t if t.dtype == torch.uint8 else t.view(torch.uint8)).numpy()


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def assert_same_bits(got: np.ndarray, want: np.ndarray, what: str) -> None:
    got = np.ascontiguousarray(got)
    want = np.ascontiguousarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    if got.dtype.itemsize == 4:
        got, want = got.view(np.uint32), want.view(np.uint32)
    bad = np.flatnonzero(got.reshape(-1) != want.reshape(-1))
    if bad.size:
        i = bad[0]
        raise AssertionError(
            f"{what}: {bad.size} of {got.size} elements differ; first at flat index {i}: "
            f"got {got.reshape(-1)[i]!r}, want {want.reshape(-1)[i]!r}"
        )

"""Operand layouts callers hand to the GEMMs (torch, any device).

These are the aiter layouts the reference's contracts declare (aklr/core/contract/semantics/_layouts.py):
- ``shuffle_weight`` -- Preshuffle(tile=(16, 16)) (:103-121): 16-row x 32-byte tiles, tile-major,
  each tile stored as two 256-byte halves (bytes 0-15 of its 16 rows, then bytes 16-31). In this layout
  the 32 lanes that feed one MFMA operand read 512 contiguous bytes. The result carries
  ``is_shuffled = True``, the tensor fact the reference's variant detection reads.
- ``shuffle_scale`` / ``e8m0_scales`` -- E8M0Scales(32, pad_to=(256, 8), shuffled=True) (:124-156): e8m0
  scales padded with 0x00 to (256, 8) multiples, then split (R/32, 2, 16, C/8, 2, 4) and permuted
  (0, 3, 5, 2, 4, 1), so one dword per lane holds 2 rows x 2 K-steps of MFMA scales.
- ``column_major`` -- ColumnMajor (:89-100): the transpose's bytes in the logical shape.
"""
from __future__ import annotations

import torch

_PRESHUFFLE_ORDER = (0, 2, 3, 1, 4)
_SCALE_ORDER = (0, 3, 5, 2, 4, 1)


def _bytes(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.uint8 else t.view(torch.uint8)


def shuffle_weight(w: torch.Tensor, layout=(16, 16)) -> torch.Tensor:
    """A [..., rows, cols] 1-byte-element weight (fp8 codes, or packed fp4 bytes) in aiter's
    shuffle_weight(layout=(16, 16)) order on the last two dims (per expert for a 3-D MoE weight);
    rows % 16 == 0, cols % 32 == 0."""
    if tuple(layout) != (16, 16):
        raise ValueError("only the (16, 16) shuffle is defined for these GEMMs")
    if w.dim() < 2 or w.element_size() != 1:
        raise ValueError("shuffle_weight takes a tensor of 1-byte elements with >= 2 dims")
    lead, (rows, cols) = tuple(w.shape[:-2]), tuple(w.shape[-2:])
    if rows % 16 or cols % 32:
        raise ValueError(f"shuffle_weight needs rows % 16 == 0 and cols % 32 == 0, got {tuple(w.shape)}")
    n = len(lead)
    order = tuple(range(n)) + tuple(n + i for i in _PRESHUFFLE_ORDER)
    x = _bytes(w).reshape(*lead, rows // 16, 16, cols // 32, 2, 16).permute(*order)
    out = x.contiguous().view(w.shape).view(w.dtype)
    out.is_shuffled = True
    return out


def unshuffle_weight(w: torch.Tensor) -> torch.Tensor:
    rows, cols = w.shape
    inv = tuple(sorted(range(5), key=_PRESHUFFLE_ORDER.__getitem__))
    split = (rows // 16, cols // 32, 2, 16, 16)
    return _bytes(w).reshape(split).permute(*inv).contiguous().view(rows, cols).view(w.dtype)


def e8m0_scales(s: torch.Tensor, shuffle: bool = True) -> torch.Tensor:
    """e8m0 scale bytes [rows, cols] -> padded to (256, 8) multiples with 0x00, shuffled."""
    b = _bytes(s)
    rows, cols = b.shape
    pr, pc = -(-rows // 256) * 256, -(-cols // 8) * 8
    stored = b.new_zeros((pr, pc))
    stored[:rows, :cols] = b
    if shuffle:
        stored = stored.reshape(pr // 32, 2, 16, pc // 8, 2, 4).permute(*_SCALE_ORDER).contiguous().view(pr, pc)
    return stored.view(s.dtype)


shuffle_scale = e8m0_scales


def column_major(t: torch.Tensor) -> torch.Tensor:
    """The transpose's bytes viewed in ``t``'s logical shape."""
    return t.mT.contiguous().view(t.shape)

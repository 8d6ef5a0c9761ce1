"""Operand layouts, restated in numpy (test infrastructure; see ``oracle/__init__.py``).

aklr/core/contract/semantics/_layouts.py:
- ``preshuffle`` (Preshuffle(tile=(16, 16)), :103-121): on a byte matrix [R, C], split
  (R/16, 16, C/32, 2, 16) and permute (0, 2, 3, 1, 4) -- 16-row x 32-byte tiles, tile-major, each tile
  as two 256-byte halves. For 1-byte elements (fp8 and packed fp4 alike) the 16-byte vector is 16 bytes.
- ``column_major`` (ColumnMajor, :89-100): the transpose's bytes viewed in the logical shape.
- ``e8m0_scales`` (E8M0Scales(32, pad_to=(256, 8), shuffled=True), :124-156): pad rows to 256 and
  columns to 8 with 0x00, then split (R/32, 2, 16, C/8, 2, 4) and permute (0, 3, 5, 2, 4, 1).
Pinned (tests/test_oracle_layouts.py) by hand-worked element positions, the inverse permutation and the
0x00 padding value (the reference's own test_padding_value, tests/core/contract/test_semantics.py:328-356).
"""
from __future__ import annotations

import numpy as np

_PRESHUFFLE_ORDER = (0, 2, 3, 1, 4)
_SCALE_ORDER = (0, 3, 5, 2, 4, 1)


def _shuffle(x: np.ndarray, split, order, inverse=False) -> np.ndarray:
    if inverse:
        split = tuple(split[i] for i in order)
        order = tuple(sorted(range(len(order)), key=order.__getitem__))
    return np.ascontiguousarray(x.reshape(split).transpose(order)).reshape(x.shape)


def preshuffle(b: np.ndarray, inverse: bool = False) -> np.ndarray:
    """uint8 [R, C] (R % 16 == 0, C % 32 == 0) -> aiter shuffle_weight(layout=(16,16)) bytes."""
    r, c = b.shape
    return _shuffle(np.ascontiguousarray(b), (r // 16, 16, c // 32, 2, 16), _PRESHUFFLE_ORDER, inverse)


def preshuffle_offset(row: int, col: int, cols: int) -> int:
    """Byte offset of element (row, col) of an [R, cols] byte matrix in the preshuffled storage."""
    return ((row // 16) * (cols // 32) + col // 32) * 512 + ((col % 32) // 16) * 256 + (row % 16) * 16 + col % 16


def column_major(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x.T).reshape(x.shape)


def e8m0_scales_storage_shape(rows: int, cols: int) -> tuple[int, int]:
    return -(-rows // 256) * 256, -(-cols // 8) * 8


def e8m0_scales(s: np.ndarray, shuffled: bool = True) -> np.ndarray:
    rows, cols = s.shape
    pr, pc = e8m0_scales_storage_shape(rows, cols)
    stored = np.zeros((pr, pc), dtype=np.uint8)
    stored[:rows, :cols] = s
    if shuffled:
        stored = _shuffle(stored, (pr // 32, 2, 16, pc // 8, 2, 4), _SCALE_ORDER)
    return stored


def e8m0_unshuffle(stored: np.ndarray, rows: int, cols: int) -> np.ndarray:
    pr, pc = stored.shape
    plain = _shuffle(stored, (pr // 32, 2, 16, pc // 8, 2, 4), _SCALE_ORDER, inverse=True)
    return plain[:rows, :cols]

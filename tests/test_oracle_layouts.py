"""Pins oracle/layouts.py and checks the product's torch layouts (aklr_amd.layouts) against it:

- Preshuffle(16, 16): hand-worked byte positions, every element against the closed-form offset
  ((row/16)*(cols/32) + col/32)*512 + ((col%32)/16)*256 + (row%16)*16 + col%16, the inverse;
- E8M0Scales(32, pad_to=(256, 8), shuffled): every element against the closed-form offset the HIP
  kernels use, and the reference's test_padding_value (tests/core/contract/test_semantics.py:336-356):
  every padded byte is 0x00 and there are exactly prod(storage) - prod(shape) of them;
- ColumnMajor: the transpose's bytes in the logical shape.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from aklr_amd import layouts as hl
from oracle import layouts as ol


def test_preshuffle_hand_worked():
    rows, cols = 32, 64
    b = np.arange(rows * cols, dtype=np.int64).reshape(rows, cols).astype(np.uint16)  # unique ids
    # use a 2-byte id split in two uint8 planes so every element is identifiable
    lo = (b & 0xFF).astype(np.uint8)
    hi = (b >> 8).astype(np.uint8)
    s_lo, s_hi = ol.preshuffle(lo).reshape(-1), ol.preshuffle(hi).reshape(-1)
    ids = s_lo.astype(np.int64) | (s_hi.astype(np.int64) << 8)
    # element (r, c) sits at offset: row tile, column tile of 32, half of 16, row in tile, byte
    assert ids[0] == 0                          # (0, 0)
    assert ids[16] == 1 * cols + 0              # (1, 0): next row of the tile, 16 bytes on
    assert ids[256] == 0 * cols + 16            # (0, 16): second 16-byte half of the first tile
    assert ids[512] == 0 * cols + 32            # (0, 32): next column tile
    assert ids[(1 * (cols // 32)) * 512] == 16 * cols  # (16, 0): next row tile
    for r in range(rows):
        for c in range(cols):
            assert ids[ol.preshuffle_offset(r, c, cols)] == r * cols + c


def test_preshuffle_inverse_and_host_layout():
    rng = np.random.default_rng(0)
    b = rng.integers(0, 256, (48, 96), dtype=np.uint8)
    s = ol.preshuffle(b)
    assert np.array_equal(ol.preshuffle(s, inverse=True), b)
    t = hl.shuffle_weight(torch.from_numpy(b))
    assert getattr(t, "is_shuffled", False) is True
    assert np.array_equal(t.numpy(), s)
    assert np.array_equal(hl.unshuffle_weight(t).numpy(), b)
    f8 = torch.from_numpy(b).view(torch.float8_e4m3fn)
    assert hl.shuffle_weight(f8).dtype == torch.float8_e4m3fn
    with pytest.raises(ValueError):
        hl.shuffle_weight(torch.from_numpy(b[:40]))


def _scale_offset(r, c, pc):
    r0, r1, r2 = r >> 5, (r >> 4) & 1, r & 15
    c0, c2, c3 = c >> 3, (c >> 2) & 1, c & 3
    return ((((r0 * (pc >> 3) + c0) * 4 + c3) * 16 + r2) * 2 + c2) * 2 + r1


@pytest.mark.parametrize("shape", [(33, 90), (3, 12), (256, 8), (300, 17)])
def test_e8m0_scales_offsets_and_padding(shape):
    rows, cols = shape
    pr, pc = ol.e8m0_scales_storage_shape(rows, cols)
    assert (pr, pc) == (-(-rows // 256) * 256, -(-cols // 8) * 8)
    ids = np.arange(rows * cols, dtype=np.int64).reshape(rows, cols)
    planes = [ol.e8m0_scales(((ids >> (8 * p)) & 0xFF).astype(np.uint8)).reshape(-1).astype(np.int64)
              for p in range(3)]
    stored_ids = planes[0] | (planes[1] << 8) | (planes[2] << 16)
    for r in range(0, rows, 7):
        for c in range(cols):
            assert stored_ids[_scale_offset(r, c, pc)] == r * cols + c
    # the reference's padding test: scales all 1 and all 2 share exactly the padding bytes, all 0x00
    ones = ol.e8m0_scales(np.full(shape, 1, np.uint8))
    twos = ol.e8m0_scales(np.full(shape, 2, np.uint8))
    padding = ones == twos
    assert padding.sum() == pr * pc - rows * cols
    assert np.all(ones[padding] == 0)
    assert np.array_equal(ol.e8m0_unshuffle(ones, rows, cols), np.full(shape, 1, np.uint8))
    host = hl.e8m0_scales(torch.from_numpy(np.full(shape, 1, np.uint8)))
    assert np.array_equal(host.numpy(), ones)


def test_column_major():
    x = np.arange(12, dtype=np.float32).reshape(3, 4)
    cm = ol.column_major(x)
    assert cm.shape == (3, 4) and np.array_equal(cm.reshape(-1), x.T.reshape(-1))
    assert np.array_equal(hl.column_major(torch.from_numpy(x)).numpy(), cm)

"""The full-size parity helpers (`tests/fullsize.py`) on the CPU: the row choice covers every
M-tile and every block position, and the accumulator checksums catch planted mistakes (one
wrong value, or two that cancel in a plain sum)."""

from __future__ import annotations

import pytest
import torch

from fullsize import checksums_exact, tile_rows


def test_tile_rows_cover_every_tile_and_block():
    rows = tile_rows(4096)
    assert len(rows) == 64
    assert set((rows // 256).tolist()) == set(range(16))
    assert set(((rows % 256) // 32).tolist()) == set(range(8))
    assert set(((rows % 256) // 128).tolist()) == {0, 1}
    ragged = tile_rows(300, 2)
    assert ragged.max() < 300 and set((ragged // 256).tolist()) == {0, 1}


def test_checksums_catch_planted_mistakes():
    gen = torch.Generator().manual_seed(1)
    q = torch.randint(-127, 128, (96, 64), generator=gen, dtype=torch.int8)
    w = torch.randint(-127, 128, (40, 64), generator=gen, dtype=torch.int8)
    acc = (q.double() @ w.double().t()).to(torch.int32)
    checksums_exact(acc, q, w, seed=2)
    one = acc.clone()
    one[17, 3] += 1
    with pytest.raises(AssertionError):
        checksums_exact(one, q, w, seed=2)
    cancel = acc.clone()  # the plain row and column sums both unchanged
    cancel[5, 7] += 1
    cancel[5, 9] -= 1
    cancel[8, 7] -= 1
    cancel[8, 9] += 1
    with pytest.raises(AssertionError):
        checksums_exact(cancel, q, w, seed=2)

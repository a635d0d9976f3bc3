"""Row choices and checksums for the full-size parity tests: which output rows to hold to the
CPU law so that every output tile of a launch is checked, and whole-matrix checks of an int32
accumulator matrix that the law fixes exactly at any size."""

from __future__ import annotations

import torch


def tile_rows(m: int, per_tile: int = 4) -> torch.Tensor:
    """Rows that cover every 256-row M-tile of an M-row GEMM, `per_tile` a tile: each from a
    different 32-row MFMA block (both 128-row wave halves), the blocks and the row within a block
    rotating from tile to tile so that every block position is seen. Each row is checked against
    every column, so every (M-tile, N-tile) output tile, and every XCD's share of the launch, is
    checked."""
    rows = []
    for t in range((m + 255) // 256):
        for i in range(per_tile):
            block = (t + 2 * i) % 8
            r = 256 * t + 32 * block + (5 * t + 11 * i) % 32
            if r < m:
                rows.append(r)
    return torch.tensor(sorted(set(rows)))


def checksums_exact(acc: torch.Tensor, q: torch.Tensor, data: torch.Tensor, seed: int) -> None:
    """The whole int32 accumulator matrix acc = q·dataᵀ [M, N] against checksums the law fixes,
    exact in int64: column sums (1ᵀq)·dataᵀ, row sums q·(dataᵀ1), and the same under random
    ±1..±7 row and column weights (so errors of opposite sign cannot cancel). A wrong value
    anywhere changes its row's and its column's sums."""
    gen = torch.Generator().manual_seed(seed)
    m, n = acc.shape
    a = acc.to(torch.int64)
    qi, wi = q.to(torch.int64), data.to(torch.int64)
    for r in (torch.ones(m, dtype=torch.int64), torch.randint(-7, 8, (m,), generator=gen)):
        assert torch.equal(r @ a, (r @ qi) @ wi.t())
    for c in (torch.ones(n, dtype=torch.int64), torch.randint(-7, 8, (n,), generator=gen)):
        assert torch.equal(a @ c, qi @ (c @ wi))

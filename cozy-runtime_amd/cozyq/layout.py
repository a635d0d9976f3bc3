"""Scale-grid layouts the leaves accept: cuBLAS's 128x4 tiled E8M0 layout (the reference's
`to_blocked` / `from_blocked`, `internal/encoding/formats.py:154-178`), converted to the
row-major `[rows, K/32]` grid the gfx950 MX GEMM reads.

In the tiled layout the grid is padded to 128-row by 4-column tiles, tiles follow one another
row-block-major, and inside a tile byte (r, c) sits at (r % 32)·16 + (r // 32)·4 + c.
"""

from __future__ import annotations

from typing import Any

Tensor = Any


def blocked_shape(rows: int, cols: int) -> tuple[int, int]:
    """The padded grid: rows up to a multiple of 128, columns up to a multiple of 4."""
    return -(-rows // 128) * 128, -(-cols // 4) * 4


def _offsets(torch: Any, rows: int, cols: int, device: Any) -> Tensor:
    """Tiled offset of every (r, c) of a `[rows, cols]` grid."""
    _, pcol = blocked_shape(rows, cols)
    r = torch.arange(rows, device=device).reshape(-1, 1)
    c = torch.arange(cols, device=device).reshape(1, -1)
    tile = (r // 128) * (pcol // 4) + c // 4
    inner = (r % 32) * 16 + ((r % 128) // 32) * 4 + c % 4
    return tile * 512 + inner


def from_blocked(torch: Any, blocked: Tensor, rows: int, cols: int) -> Tensor:
    """The row-major `[rows, cols]` grid of a tiled one."""
    flat = blocked.reshape(-1)
    prow, pcol = blocked_shape(rows, cols)
    if flat.numel() != prow * pcol:
        raise ValueError(f"a 128x4 tiled grid of [{rows}, {cols}] holds {prow * pcol} bytes, "
                         f"not {flat.numel()}")  # fmt: skip
    return flat[_offsets(torch, rows, cols, flat.device)].contiguous()


def to_blocked(torch: Any, grid: Tensor) -> Tensor:
    """The tiled layout of a row-major `[rows, cols]` grid (padding bytes zero)."""
    rows, cols = int(grid.shape[0]), int(grid.shape[1])
    prow, pcol = blocked_shape(rows, cols)
    out = torch.zeros(prow * pcol, dtype=grid.dtype, device=grid.device)
    out[_offsets(torch, rows, cols, grid.device).reshape(-1)] = grid.reshape(-1)
    return out

"""Argument admission for the op library (`cozyq.prebuilt`), as data.

Each operand an op takes is described by an `Operand`: the dtypes it may have, its extents (which
also fix its rank) or element count, whether it must be dense, its byte alignment, a multiple its
first extent must be, and an element size. `faults` lists the properties a tensor breaks, in the
fixed order of `PROPERTIES`. An op pairs each operand with a `Messages` table, from property to
the text the reference's op library raises for it (the contract: `internal/prebuilt.py:360-406`,
`:193-250`, `:263-291`), and `admit` raises ValueError with the first fault's text. Cards are
checked separately (`off_card`), after every operand's own properties, as the contract orders it.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

Tensor = Any

KIND, EXTENT, LAYOUT, ALIGN, ROWS = "kind", "extent", "layout", "align", "rows"
#: The order properties are checked in; an operand's first fault names the error.
PROPERTIES = (KIND, EXTENT, LAYOUT, ALIGN, ROWS)


@dataclass(frozen=True)
class Operand:
    """What one tensor argument must be. `extents`: one entry a dimension, None where any extent
    goes (the tuple's length is the rank); `count`: the element count, whatever the shape."""

    kinds: tuple[Any, ...] = ()
    extents: tuple[int | None, ...] | None = None
    count: int | None = None
    dense: bool = False
    align: int = 1
    rows: int = 1
    itemsize: int | None = None


Messages = dict[str, str]


def faults(t: Tensor, spec: Operand) -> list[str]:
    """The properties of `spec` that `t` breaks, in `PROPERTIES` order (each at most once)."""
    broken: set[str] = set()
    if (spec.kinds and t.dtype not in spec.kinds) or (
        spec.itemsize is not None and t.element_size() != spec.itemsize
    ):
        broken.add(KIND)
    if spec.extents is not None:
        if t.dim() != len(spec.extents) or any(
            want is not None and got != want for got, want in zip(t.shape, spec.extents)
        ):
            broken.add(EXTENT)
    if spec.count is not None and t.numel() != spec.count:
        broken.add(EXTENT)
    if spec.dense and not t.is_contiguous():
        broken.add(LAYOUT)
    if spec.align > 1 and t.data_ptr() % spec.align:
        broken.add(ALIGN)
    if spec.rows > 1 and (t.dim() == 0 or t.shape[0] % spec.rows):
        broken.add(ROWS)
    return [p for p in PROPERTIES if p in broken]


def admit(*checks: tuple[Tensor, Operand, Messages]) -> None:
    """Raises ValueError with the message of the first fault, operand by operand."""
    for t, spec, says in checks:
        found = faults(t, spec)
        if found:
            raise ValueError(says[found[0]])


def every(text: str, *properties: str) -> Messages:
    """One message for each of `properties` (all of them when none are named)."""
    return {p: text for p in (properties or PROPERTIES)}


def off_card(index: int, *tensors: Tensor | None) -> bool:
    """Whether any of the given tensors is not on cuda:`index`."""
    return any(t is not None and (not t.is_cuda or t.get_device() != index) for t in tensors)


@dataclass(frozen=True)
class Placement:
    """Where the GEMM may write its `[rows, n]` result in place: a tensor of the output dtype on
    the op's device, the last axis dense and rows at least `n` elements apart, a whole number of
    16-byte units apart and starting at a 16-byte address (the stores are 16 bytes wide)."""

    rows: int
    n: int
    dtype: Any
    device: Any
    unit: int = field(default=16)

    def takes(self, out: Tensor) -> bool:
        if out.dtype != self.dtype or out.device != self.device or tuple(out.shape) != (self.rows, self.n):
            return False
        row_step, col_step = out.stride()
        return (col_step == 1 and row_step >= self.n and (row_step * out.element_size()) % self.unit == 0
                and out.data_ptr() % self.unit == 0)  # fmt: skip

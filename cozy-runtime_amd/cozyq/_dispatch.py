"""What every per-format op module checks before it launches, and how a result reaches `out`.

The kernels are the only implementation. An operand off the GPU, or an activation or output
that is not 16-bit, raises ValueError naming the op. It never takes a slower path.
"""

from __future__ import annotations

from typing import Any

from cozyq import prebuilt

Tensor = Any
Dtype = Any


def library(index: int) -> prebuilt.Prebuilt:
    """The op library of card `index` (opened once per process by `prebuilt.library`)."""
    return prebuilt.library(index)


def card(op: str, x: Tensor) -> int:
    """The index of the card holding `x`; a ValueError if `x` is not on one."""
    if x.is_cuda:
        return x.get_device()
    raise ValueError(f"{op}: the operand is on {x.device}; the kernels run on a gfx950 card")


def sixteen_bit(op: str, torch: Any, *dtypes: Dtype) -> None:
    """A ValueError unless every one of `dtypes` is bf16 or fp16."""
    for dtype in dtypes:
        if dtype is not torch.bfloat16 and dtype is not torch.float16:
            raise ValueError(f"{op}: activations and outputs are bf16 or fp16, not {dtype}")


def activation_card(op: str, torch: Any, x: Tensor, *out_dtypes: Dtype) -> int:
    """`card(op, x)` for a 16-bit activation `x` whose outputs are `out_dtypes`."""
    index = card(op, x)
    sixteen_bit(op, torch, x.dtype, *out_dtypes)
    return index


def out_rows(out: Tensor | None, n: int) -> Tensor | None:
    """The `[M, n]` view a GEMM writes for a caller's `out`, or None when `out`'s rows cannot
    be viewed so. The caller's result is then copied in afterwards."""
    if out is not None:
        try:
            return out.view(-1, n)
        except RuntimeError:
            pass
    return None


def deliver(result: Tensor, out: Tensor | None) -> Tensor:
    """`result`, or `out` holding it when the caller passed one. A GEMM that wrote into `out`'s
    storage needs no copy."""
    if out is not None and result.data_ptr() != out.data_ptr():
        out.copy_(result)
    return result if out is None else out

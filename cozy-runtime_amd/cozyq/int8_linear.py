"""The int8.convrot linear's ops on gfx950 — cozyq's counterpart of cozy-runtime's
`internal/int8_linear.py` (`linear`, `quantize`, `prologue`, `gemm`, `into`, `landed`,
`serving`), with the same names, arguments and return conventions.

One difference is deliberate: the reference falls back to comfy-kitchen's kernels or to torch's
eager int8 GEMM when its op does not serve a call; here the HIP kernels are the only
implementation, so a tensor they cannot take (not on a gfx950 card, not bf16/fp16) raises
instead of running elsewhere, and a missing library raises `KernelsAbsent`.
"""

from __future__ import annotations

from typing import Any

from cozyq import prebuilt
from cozyq.operands import INT8_CONVROT, PreQuantized

Tensor = Any
Dtype = Any

#: The op's name in a run's `gemm.selected` (`internal/int8_linear.py:41`).
OP = "cozy-int8"
#: Rows a GEMV launch serves (`internal/int8_linear.py:45`, `int8.h:20`).
GEMV_ROWS = 4
#: The quantize kernel's prologue codes (`internal/int8_linear.py:302-305`).
NORMS = {None: 0, "layer": 1, "rms": 2}
ACTIVATIONS = {None: 0, "gelu": 1, "gelu_tanh": 2, "situ": 3, "swiglu": 4}
GATED = frozenset({"situ"})

_LIBS: dict[int, prebuilt.Prebuilt] = {}


def library(index: int) -> prebuilt.Prebuilt:
    """The op library on card `index`, opened once (`internal/int8_linear.py:100-103`)."""
    lib = _LIBS.get(index)
    if lib is None:
        lib = _LIBS[index] = prebuilt.library(index)
    return lib


def _card(x: Tensor) -> int:
    """The card index of a device operand, or a ValueError naming where it is instead."""
    if not x.is_cuda:
        raise ValueError(f"{OP}: the operand is on {x.device}; the kernels run on a gfx950 card")
    return x.get_device()


def _half(torch: Any, *dtypes: Dtype) -> None:
    """A ValueError unless each of `dtypes` is bf16 or fp16 (the kernels' 16-bit types)."""
    for dtype in dtypes:
        if dtype not in (torch.bfloat16, torch.float16):
            raise ValueError(f"{OP}: activations and outputs are bf16 or fp16, not {dtype}")


def _served(torch: Any, x: Tensor, *dtypes: Dtype) -> int:
    """`_card(x)` for 16-bit `x`, with each of `dtypes` 16-bit too."""
    index = _card(x)
    _half(torch, x.dtype, *dtypes)
    return index


def linear(torch: Any, x: Tensor, data: Tensor, scale: Tensor, bias: Tensor | None,
           out_dtype: Dtype) -> Tensor:  # fmt: skip
    """`x @ W.T + bias` for one int8.convrot (rotation 256) weight: `data` int8 `[N, K]`,
    `scale` float32 `[N]` (`internal/int8_linear.py:244-276`)."""
    index = _served(torch, x, out_dtype)
    return library(index).int8_linear(x, data, scale, bias, out_dtype)


def serving(index: int) -> str:
    """The kernel this card's int8 leaves serve (`internal/int8_linear.py:279-283`)."""
    library(index)
    return OP


def quantize(torch: Any, x: Tensor) -> PreQuantized | None:
    """`x` rotated and quantized once for several int8 leaves (`internal/int8_linear.py:
    286-299`), or None for the GEMV's few rows, which each leaf's own call serves."""
    index = _served(torch, x)
    if x.numel() <= GEMV_ROWS * x.shape[-1]:
        return None
    payload, scale = library(index).int8_quantize(x)
    return PreQuantized(payload, scale, tuple(x.shape), INT8_CONVROT)


def prologue(
    torch: Any,
    x: Tensor,
    consumers: tuple[object, ...],
    *,
    norm: str | None,
    eps: float,
    scale: Tensor | None,
    shift: Tensor | None,
    activation: str | None,
    up: Tensor | None = None,
) -> PreQuantized | None:
    """`activation(norm(x)·(1 + scale) + shift)` rotated and quantized in one pass
    (`internal/int8_linear.py:308-357`) when each of `consumers` is an un-hooked leaf of the
    rows' width taking int8.convrot's operand; else None and the caller runs its own ops. The
    reference's argument rules hold: a gated activation (`GATED`, or swiglu without `up`) reads
    x's [hidden | gate] halves alone; `up` only with swiglu, of x's shape."""
    gated = activation in GATED or (activation == "swiglu" and up is None)
    if gated and (norm is not None or scale is not None or shift is not None or x.shape[-1] % 2):
        raise ValueError(f"int8_rows: {activation} takes [hidden | gate] rows, no norm or tables")
    if up is not None and (
        activation != "swiglu" or norm is not None or scale is not None or shift is not None
    ):
        raise ValueError("int8_rows: swiglu takes gate and up rows, no norm or tables")
    if norm not in NORMS or activation not in ACTIVATIONS:
        raise ValueError(f"int8_rows: norm {norm!r} / activation {activation!r} unknown")
    if up is not None and (up.shape != x.shape or up.dtype != x.dtype or not up.is_cuda):
        return None
    width = x.shape[-1] // 2 if gated else x.shape[-1]
    if not x.is_cuda or x.dtype not in (torch.bfloat16, torch.float16):
        return None
    if any(t is not None and t.dtype != x.dtype for t in (scale, shift)):
        return None  # eager promotes the rows to the table's dtype
    hooks = torch.nn.modules.module
    if hooks._global_forward_hooks or hooks._global_forward_pre_hooks:
        return None
    for module in consumers:
        if getattr(module, "operand", None) != INT8_CONVROT or getattr(module, "in_features", None) != width:
            return None
        if not _inert(module):
            return None
    payload, row_scale = library(x.get_device()).int8_quantize(
        x, scale, shift, NORMS[norm], eps, ACTIVATIONS[activation], up
    )
    return PreQuantized(payload, row_scale, (*x.shape[:-1], width), INT8_CONVROT)


def _inert(module: object) -> bool:
    """No hook of `module`'s changes its forward now (`internal/int8_linear.py:360-369`)."""
    if getattr(module, "_forward_pre_hooks", None):
        return False
    for hook in getattr(module, "_forward_hooks", {}).values():
        armed = getattr(hook, "armed", None)
        if not (getattr(hook, "_cozy_baked", False) or (armed is not None and armed() is None)):
            return False
    return True


def gemm(torch: Any, operand: PreQuantized, data: Tensor, scale: Tensor, bias: Tensor | None,
         out_dtype: Dtype, out: Tensor | None = None) -> Tensor:  # fmt: skip
    """The linear of a `quantize`d operand: the GEMM with both scales and the bias in its
    epilogue, into `out` where given (`internal/int8_linear.py:372-392`)."""
    if operand.payload.dtype != torch.int8:
        raise ValueError(f"{OP}: the operand payload must be int8, not {operand.payload.dtype}")
    index = _card(operand.payload)
    _half(torch, out_dtype)
    rows = into(out, data.shape[0])
    result = library(index).int8_gemm(operand.payload, operand.scale, data, scale, bias,
                                      out_dtype, out=rows)  # fmt: skip
    return landed(result.view(*operand.shape[:-1], -1), out)


def into(out: Tensor | None, n: int) -> Tensor | None:
    """`out`'s rows as the `[M, n]` view a GEMM writes, None where they do not flatten
    (`internal/int8_linear.py:395-403`)."""
    if out is None:
        return None
    try:
        return out.view(-1, n)
    except RuntimeError:
        return None


def landed(result: Tensor, out: Tensor | None) -> Tensor:
    """`result`, in `out` where one was given (`internal/int8_linear.py:406-412`)."""
    if out is None:
        return result
    if result.data_ptr() != out.data_ptr():
        out.copy_(result)
    return out

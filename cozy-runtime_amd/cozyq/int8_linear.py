"""The int8.convrot op on gfx950, under the module and function names of cozy-runtime's
`internal/int8_linear.py`: `linear`, `quantize`, `prologue`, `gemm`, `serving`.

Unlike the reference there is no fallback to comfy-kitchen or to torch's int8 GEMM. An
operand the kernels cannot take (off a gfx950 card, or not 16-bit) raises ValueError, and a
missing library raises `KernelsAbsent`. The producer prologue is admitted by rules P1–P3: the
argument refusals first, then the conditions under which the caller runs its own ops.
"""

from __future__ import annotations

from typing import Any

from cozyq import _dispatch
from cozyq.operands import INT8_CONVROT, PreQuantized

Tensor = Any
Dtype = Any

#: The op's name in a run's `gemm.selected` (`internal/int8_linear.py:41`).
OP = "cozy-int8"
#: Rows the one-launch GEMV takes (`internal/int8_linear.py:45`).
GEMV_ROWS = 4
#: The quantize kernel's prologue codes (`internal/int8_linear.py:302-305`).
NORMS = {None: 0, "layer": 1, "rms": 2}
ACTIVATIONS = {None: 0, "gelu": 1, "gelu_tanh": 2, "situ": 3, "swiglu": 4}
#: Activations that read [hidden | gate] halves of x (and SwiGLU without `up` rows).
GATED = frozenset({"situ"})


def library(index: int) -> Any:
    return _dispatch.library(index)


def linear(torch: Any, x: Tensor, data: Tensor, scale: Tensor, bias: Tensor | None,
           out_dtype: Dtype) -> Tensor:  # fmt: skip
    """`x @ Wᵀ + bias` for an int8.convrot weight (rotation 256): `data` int8 `[N, K]`,
    `scale` float32 `[N]` (`internal/int8_linear.py:244-276`). Up to `GEMV_ROWS` rows take the
    fused GEMV; more are quantized, then multiplied."""
    index = _dispatch.activation_card(OP, torch, x, out_dtype)
    return library(index).int8_linear(x, data, scale, bias, out_dtype)


def serving(index: int) -> str:
    """The op this card's int8 leaves run (`internal/int8_linear.py:279-283`)."""
    library(index)
    return OP


def quantize(torch: Any, x: Tensor) -> PreQuantized | None:
    """`x` rotated and quantized once, for every int8 leaf reading it
    (`internal/int8_linear.py:286-299`). None for as few rows as the GEMV takes: each leaf's own
    call then runs the fused GEMV."""
    index = _dispatch.activation_card(OP, torch, x)
    if x.numel() > GEMV_ROWS * x.shape[-1]:
        payload, scale = library(index).int8_quantize(x)
        return PreQuantized(payload, scale, tuple(x.shape), INT8_CONVROT)
    return None


def gemm(torch: Any, operand: PreQuantized, data: Tensor, scale: Tensor, bias: Tensor | None,
         out_dtype: Dtype, out: Tensor | None = None) -> Tensor:  # fmt: skip
    """The linear of a quantized operand, with both scales and the bias in the GEMM's epilogue.
    The result is written into `out` when it is given (`internal/int8_linear.py:372-392`)."""
    if operand.payload.dtype is not torch.int8:
        raise ValueError(f"{OP}: the operand payload must be int8, not {operand.payload.dtype}")
    index = _dispatch.card(OP, operand.payload)
    _dispatch.sixteen_bit(OP, torch, out_dtype)
    written = library(index).int8_gemm(operand.payload, operand.scale, data, scale, bias, out_dtype,
                                       out=_dispatch.out_rows(out, data.shape[0]))  # fmt: skip
    return _dispatch.deliver(written.view(*operand.shape[:-1], -1), out)


# ------------------------------------------------------------ the producer prologue


def _refusal(x: Tensor, norm: str | None, scale: Tensor | None, shift: Tensor | None,
             activation: str | None, up: Tensor | None) -> str | None:  # fmt: skip
    """P1: the message of an argument set the prologue refuses, or None."""
    tables = norm is not None or scale is not None or shift is not None
    if activation in GATED or (activation == "swiglu" and up is None):
        if tables or x.shape[-1] % 2:
            return f"int8_rows: {activation} takes [hidden | gate] rows, no norm or tables"
    if up is not None and (activation != "swiglu" or tables):
        return "int8_rows: swiglu takes gate and up rows, no norm or tables"
    if norm not in NORMS or activation not in ACTIVATIONS:
        return f"int8_rows: norm {norm!r} / activation {activation!r} unknown"
    return None


def _quiet(module: object) -> bool:
    """No hook changes `module`'s forward now: it has no forward pre-hook, and each forward
    hook is either baked into the leaf (`_cozy_baked`) or disarmed (`armed()` is None)."""
    if getattr(module, "_forward_pre_hooks", None):
        return False
    for hook in getattr(module, "_forward_hooks", {}).values():
        if getattr(hook, "_cozy_baked", False):
            continue
        armed = getattr(hook, "armed", None)
        if armed is None or armed() is not None:
            return False
    return True


def _declines(torch: Any, x: Tensor, consumers: tuple[object, ...], width: int,
              scale: Tensor | None, shift: Tensor | None, up: Tensor | None) -> bool:  # fmt: skip
    """P2: whether the caller must run its own ops instead."""
    if up is not None and (up.shape != x.shape or up.dtype != x.dtype or not up.is_cuda):
        return True
    if not x.is_cuda or x.dtype not in (torch.bfloat16, torch.float16):
        return True
    if any(table is not None and table.dtype != x.dtype for table in (scale, shift)):
        return True  # an eager prologue would promote the rows to the table's dtype
    registry = torch.nn.modules.module
    if registry._global_forward_hooks or registry._global_forward_pre_hooks:
        return True
    return not all(getattr(m, "operand", None) == INT8_CONVROT and getattr(m, "in_features", None) == width
                   and _quiet(m) for m in consumers)  # fmt: skip


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
    """`activation(norm(x)·(1 + scale) + shift)` rotated and quantized in one pass, for
    `consumers` that all take int8.convrot's operand (`internal/int8_linear.py:308-357`).
    Admission follows P1–P3: a ValueError for a refused argument set, None where the caller
    runs its own ops, else the operand (half of x's width for the gated forms)."""
    why = _refusal(x, norm, scale, shift, activation, up)
    if why is not None:
        raise ValueError(why)
    gated = activation in GATED or (activation == "swiglu" and up is None)
    width = x.shape[-1] // 2 if gated else x.shape[-1]
    if _declines(torch, x, consumers, width, scale, shift, up):
        return None
    payload, row_scale = library(x.get_device()).int8_quantize(
        x, scale, shift, NORMS[norm], eps, ACTIVATIONS[activation], up)  # fmt: skip
    return PreQuantized(payload, row_scale, (*x.shape[:-1], width), INT8_CONVROT)

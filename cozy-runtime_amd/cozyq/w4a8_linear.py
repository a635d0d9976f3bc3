"""The `w4a8.convrot` encoded GEMM's ops on gfx950 — cozyq's counterpart of cozy-runtime's
`internal/w4a8_linear.py` (`linear`, `gemm`): 4-bit codes in int8.convrot's rotated basis,
unpacked to int8 levels on the way to the int8 MFMA and multiplied with int8.convrot's
activation operand (quantized by the int8 leaves' op and shared with them).

As for every op here, the HIP kernels are the only implementation: the reference's torch-ops
slow path (unpack, then the int8 lane's GEMM) is the many-row config of `Prebuilt.w4a8_gemm`
itself, on the GPU.
"""

from __future__ import annotations

from typing import Any

from cozyq import _dispatch, prebuilt
from cozyq.operands import INT8_CONVROT, PreQuantized

Tensor = Any
Dtype = Any

#: The op's name in a run's `gemm.selected` (`internal/w4a8_linear.py:20`).
OP = "cozy-w4a8"
#: The activation operand it takes: int8.convrot's.
OPERAND = INT8_CONVROT


def linear(torch: Any, x: Tensor, w: prebuilt.W4a8, bias: Tensor | None, out_dtype: Dtype) -> Tensor:
    """`x @ W.T + bias` for one w4a8 weight (`internal/w4a8_linear.py:72-84`)."""
    index = _dispatch.activation_card(OP, torch, x, out_dtype)
    return _dispatch.library(index).w4a8_linear(x, w, bias, out_dtype)


def gemm(torch: Any, operand: PreQuantized, w: prebuilt.W4a8, bias: Tensor | None,
         out_dtype: Dtype, out: Tensor | None = None) -> Tensor:  # fmt: skip
    """The linear of an int8.convrot operand (`int8_linear.quantize`, a producer's prologue),
    copied into `out` where given (`internal/w4a8_linear.py:87-107`)."""
    if operand.provider != INT8_CONVROT or operand.payload.dtype != torch.int8:
        raise ValueError(f"{OP}: the operand must be int8.convrot's, not {operand.provider}")
    index = _dispatch.card(OP, operand.payload)
    _dispatch.sixteen_bit(OP, torch, out_dtype)
    result = _dispatch.library(index).w4a8_gemm(operand.payload, operand.scale, w, bias, out_dtype)
    return _dispatch.deliver(result.view(*operand.shape[:-1], -1), out)


def serving(index: int) -> str:
    """The kernel this card's w4a8 leaves serve (`internal/w4a8_linear.py:64-69`)."""
    _dispatch.library(index)
    return OP

"""The fp8.rowwise linear's ops on gfx950 — cozyq's counterpart of cozy-runtime's
`internal/fp8_linear.py` (`quantize`, `gemm`, `linear`, `serving`).

As for every op here, the HIP kernels are the only implementation: where the reference falls
back to torch ops and `_scaled_mm`, a tensor the kernels cannot take raises.
"""

from __future__ import annotations

from typing import Any

from cozyq import _dispatch
from cozyq.operands import ROWWISE_FP8, PreQuantized

Tensor = Any
Dtype = Any

#: The op's name in a run's `gemm.selected` (`internal/fp8_linear.py:27`).
OP = "cozy-fp8"
#: A derived scale's floor and E4M3's largest finite value (`internal/fp8_linear.py:24`,
#: `internal/encoding/formats.py:497`).
SCALE_FLOOR = 1e-12
E4M3_MAX = 448.0


def quantize(torch: Any, x: Tensor) -> PreQuantized:
    """`x` as the fp8 leaves' shared operand (`internal/fp8_linear.py:66-75`): E4M3 `[M, K]`
    and per-row float32 scales amax/448."""
    index = _dispatch.activation_card(OP, torch, x)
    payload, scale = _dispatch.library(index).fp8_quantize(x)
    return PreQuantized(payload, scale, tuple(x.shape), ROWWISE_FP8)


def gemm(torch: Any, operand: PreQuantized, data: Tensor, scale: Tensor, bias: Tensor | None,
         out_dtype: Dtype, out: Tensor | None = None) -> Tensor:  # fmt: skip
    """The linear of a quantized operand: the fp8 GEMM with both scales and the bias in its
    epilogue, into `out` where given (`internal/fp8_linear.py:78-111`)."""
    if operand.payload.dtype != torch.float8_e4m3fn:
        raise ValueError(f"{OP}: the operand payload must be E4M3, not {operand.payload.dtype}")
    index = _dispatch.card(OP, operand.payload)
    _dispatch.sixteen_bit(OP, torch, out_dtype)
    result = _dispatch.library(index).fp8_gemm(
        operand.payload, operand.scale, data, scale, bias, out_dtype,
        out=_dispatch.out_rows(out, data.shape[0]),
    )  # fmt: skip
    return _dispatch.deliver(result.view(*operand.shape[:-1], -1), out)


def linear(torch: Any, x: Tensor, data: Tensor, scale: Tensor, bias: Tensor | None,
           out_dtype: Dtype) -> Tensor:  # fmt: skip
    """`x @ W.T + bias` for one fp8.rowwise weight: `data` E4M3 `[N, K]`, `scale` float32
    (`internal/fp8_linear.py:114-129`); up to 16 rows in one fused launch."""
    index = _dispatch.activation_card(OP, torch, x, out_dtype)
    return _dispatch.library(index).fp8_linear(x, data, scale, bias, out_dtype)


def serving(index: int) -> str:
    """The GEMM this card's fp8 leaves serve (`internal/fp8_linear.py:132-141`)."""
    _dispatch.library(index)
    return OP

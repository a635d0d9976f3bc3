"""The `svdq.nvfp4` linear on gfx950: cozyq's counterpart of cozy-runtime's
`internal/svdq_linear.py`.

`y = (q(x · p) · Wᵀ) · g_x · g_w · c + (x · downᵀ) · upᵀ + bias`, the reference's law, on three
launches of the library: the activation's second level g_x (`cozyq_svdq_input_scale`, skipped for
a stored `input_scale`), the activation side (`cozyq_svdq_quantize`: nvfp4 codes and E4M3 block
scales of bf16(x·p), and the low-rank input bf16(x·downᵀ), from one read of x) and the GEMM
(`cozyq_svdq_gemm`: both operands decoded exactly to fp16 on the matrix core, the low-rank term
in the same accumulators, c and the bias in the epilogue, one rounding).

The weight stays as stored: codes `[N, K/2]` with element 2k low and row-major E4M3 scales
`[N, K/16]` (the reference retiles them for its RTX 50 kernel; this GEMM reads them as they
are). There is no Triton or eager lane: an activation off the GPU, or not 16-bit, raises.
"""

from __future__ import annotations

from collections.abc import Mapping
from typing import Any

from cozyq import _dispatch

Tensor = Any
Dtype = Any

#: E4M3's largest finite value times E2M1's (`internal/svdq_linear.py:44`).
LEVELS_MAX = 448.0 * 6.0
#: E4M3's least subnormal: the block-scale floor (`internal/svdq_linear.py:46`).
SCALE_FLOOR = 2.0**-9
#: The ranks the kernels are built for; a branch is padded with zero rows to the next one
#: (`internal/svdq_linear.py:49`).
RANKS = (32, 64, 128)
#: The column multiple the kernels need: one 64-element K step of the GEMM.
K_ALIGN = 64
#: The rows the activation operand is padded to (`internal/svdq_linear.py:59`).
NATIVE_ROWS = 256
#: What a run's `gemm.selected` names for these kernels.
NATIVE = "cozyq-svdq-nvfp4-mfma"


def rank(r: int) -> int:
    """Contract R1: the least built rank that holds `r` ranks (`internal/svdq_linear.py:266-271`);
    a branch past the largest raises ValueError."""
    fits = [built for built in RANKS if built >= r]
    if not fits:
        raise ValueError(f"a low-rank branch of rank {r} exceeds the kernels' {RANKS[-1]}")
    return fits[0]


def _branch(torch: Any, parts: list[tuple[Tensor, Tensor]]) -> tuple[Tensor, Tensor]:
    """The factors (down [r_i, K], up [N, r_i]) laid end to end in one bf16 branch of the least
    built rank that holds them all, the ranks past their sum zero (they add nothing to
    `la·upᵀ`): each factor is copied into its slice of a zeroed buffer, rounded to bf16 on the way."""
    total = sum(int(d.shape[0]) for d, _ in parts)
    width = rank(total)
    first_down, first_up = parts[0]
    down = torch.zeros(width, first_down.shape[1], dtype=torch.bfloat16, device=first_down.device)
    up = torch.zeros(first_up.shape[0], width, dtype=torch.bfloat16, device=first_up.device)
    at = 0
    for d, u in parts:
        r = int(d.shape[0])
        down[at:at + r].copy_(d)
        up[:, at:at + r].copy_(u)
        at += r
    return down, up


def padded(torch: Any, down: Tensor, up: Tensor) -> tuple[Tensor, Tensor]:
    """Contract R2 (`internal/svdq_linear.py:274-283`): a branch `(down [r, K], up [N, r])` as
    contiguous bf16 of rank `rank(r)`, zero past r."""
    return _branch(torch, [(down, up)])


def merged(torch: Any, roles: Mapping[str, Tensor], down: Tensor, up: Tensor) -> dict[str, Tensor] | None:
    """Contract R3 (`internal/svdq_linear.py:286-299`): the low-rank roles with a LoRA's
    factors appended as more ranks, so `x·downᵀ·upᵀ` gains `x·Aᵀ·(s·B)ᵀ` with no rounding of
    the weight; None when the ranks together pass the kernels' largest (the caller then adds the
    LoRA's term itself)."""
    own_down, own_up = roles["lowrank_down"], roles["lowrank_up"]
    if int(own_down.shape[0]) + int(down.shape[0]) > RANKS[-1]:
        return None
    both, wide = _branch(torch, [(own_down, own_up), (down, up)])
    return {"lowrank_down": both, "lowrank_up": wide}


def serving(index: int) -> str:
    """The kernel this card's svdq leaves run (`internal/svdq_linear.py:443-448`)."""
    _dispatch.library(index)
    return NATIVE


def linear(torch: Any, x: Tensor, roles: Mapping[str, Tensor], bias: Tensor | None,
           out_dtype: Dtype) -> Tensor:  # fmt: skip
    """`x @ Wᵀ + bias` for one leaf's roles (`internal/svdq_linear.py:662-697`): `weight` u8
    `[N, K/2]`, `scale` E4M3 `[N, K/16]`, `scale_2` f32, `pre_quant_scale` f32 `[K]`,
    `lowrank_down` bf16 `[R, K]` and `lowrank_up` bf16 `[N, R]` (R one of `RANKS`), optional
    `channel_scale` `[N]` and `input_scale`. x and the output are bf16 or fp16, each its own
    (the GEMM rounds once, into `out_dtype`)."""
    index = _dispatch.activation_card("svdq", torch, x, out_dtype)
    return _dispatch.library(index).svdq_linear(x, dict(roles), bias, out_dtype)

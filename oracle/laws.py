"""CPU restatement of the quantized-linear laws — TEST INFRASTRUCTURE ONLY (see `oracle/__init__`).

Every function restates one law of cozy-runtime (`/root/reference`, cited `path:line`, paths
relative to `src/cozy_runtime/`) in torch CPU ops, operation for operation, so that the float32
rounding sequence is the reference's. Where this build adds a law the reference lacks (the
128-channel rotation, the rotation-off int8 lane, the tanh-GELU epilogue, the int4-g64 SVDQuant
variant), the docstring says "build law" and names what pins it.

Pins, exercised in `tests/test_oracle.py`:
- `hadamard` (256): the reference's int8.convrot decode vectors (signs and index order) and the
  closed form H·H = n·I; float32 association order: the expression text at
  `internal/encoding/formats.py:667-671`, which the code below evaluates left to right.
- `e4m3`, `e8m0_multipliers`, `to_blocked`/`from_blocked`: the reference's fp8 and mxfp8 decode
  vectors, plus an independent bit-level e4m3 encoder checked over every bf16/fp16 input.
- `mx_quantize`: brute force over every positive bf16 and fp16 block maximum (exact integer ceil
  of log2) and the round trip through the mxfp8 decode law.
- `int8_*` products: int32 GEMM against numpy int64 matmul; `int8_epilogue`'s float sequence
  (accumulator to float32, `· xs`, `· ws`, the cast, the bias in the output dtype) against
  exact rational arithmetic with an independent round-to-nearest-even, on cases where each
  plausible reordering gives other bits.
- `gelu_tanh` (build law for the C2 epilogue): torch's tanh-approximate GELU in float64 over
  every bf16 value in [-12, 12], bounded by the formula's own cancellation; zero and the
  odd-part identity.
- `int4_quantize` (build law): round trip bound |x − q·s| ≤ s/2 and brute force on small cases.
- `w4a8_unpack`: closed forms (unit group scale on the uniform grid gives q − 8, the nibble
  order, NaN scales, the ±127 clamp) and numpy's float32 multiply and `rint` over every
  (scale byte, code) pair.
- `prologue` (the producer prologue, compared with tolerance on the GPU since its
  transcendentals are the platform's): closed forms (constant and alternating rows through
  each norm, unit / zero modulation, table-row selection) and the library routines `math.erf`,
  `math.tanh`, `math.exp` and `torch.nn.functional.silu` on scalars.
- `svdq_smooth`, `svdq_down`, `svdq_exact` (the W4A4 structure): closed forms — unit and
  power-of-two smoothing, one-hot and integer-valued down projections (against numpy int64),
  the fp16 cast of `down` for fp16 x, and activations/weights placed on the int4 grid so that
  the product equals numpy's matmul of the dequantized operands, group by group.
- `svdq_nvfp4_quantize` (svdq.nvfp4's activation law): its E2M1 threshold count against
  brute-force nearest-E2M1 with ties to the even code over a dense sweep and every midpoint with
  its float32 neighbours, both signs (-0 keeps code 0); the block scale against the independent
  bit encoder, the 2^-9 floor of an all-zero block and the 448 saturation; the decode round trip
  within half an E2M1 step. `svdq_nvfp4_input_scale`: element-by-element numpy float32 brute
  force, the zero floor and a stored scale. `svdq_nvfp4_exact`: on-grid activations (lossless
  quantization) against the golden-pinned `decode_nvfp4` weight, c, a one-hot low-rank branch
  and the bias.
"""

from __future__ import annotations

import math

import numpy as np
import torch

#: E4M3's largest finite magnitude (`internal/encoding/formats.py:497`).
E4M3_MAX = 448.0
#: A derived scale's floor (`internal/fp8_linear.py:24`, `internal/int8_linear.py:426`).
SCALE_FLOOR = 1e-12
#: MX block along K (`internal/encoding/formats.py:118`).
MX_BLOCK = 32
#: The reference's rotation sizes `4**k` (`internal/encoding/formats.py:661`); 128 is this
#: build's extension (H2 ⊗ H4 ⊗ H4 ⊗ H4).
ROTATION_SIZES = tuple(4**k for k in range(1, 9))
#: int4 SVDQuant variant: K-group and code range (build law).
INT4_GROUP = 64
INT4_MAX = 7.0


# ----------------------------------------------------------------------------- rotation


def _digits(size: int) -> list[int]:
    """The radices of the rotation's stages, outer digit first."""
    if size in ROTATION_SIZES:
        return [4] * ROTATION_SIZES.index(size) + [4]
    if size == 128:
        return [2, 4, 4, 4]
    raise ValueError(f"rotation size {size} is neither 4**k nor 128")


def hadamard(x: torch.Tensor, size: int) -> torch.Tensor:
    """Each `size`-group of the last axis times the unnormalized Hadamard, one stage per digit,
    outer digit first (`internal/encoding/formats.py:657-671`; numpy twin
    `derive/microscale.py:272-282`). A 4-point stage maps (a, b, c, d) to
    (a+b+c-d, a+b-c+d, a-b+c+d, b+c+d-a), each evaluated left to right in x's dtype. Size 128
    (build law) puts the Sylvester 2-point stage (a+b, a-b) first, then three 4-point stages."""
    shape = x.shape
    digits = _digits(size)
    work = x.reshape(-1, *digits)
    for axis in range(1, len(digits) + 1):
        parts = work.unbind(axis)
        if len(parts) == 4:
            a, b, c, d = parts
            out = (a + b + c - d, a + b - c + d, a - b + c + d, b + c + d - a)
        else:
            a, b = parts
            out = (a + b, a - b)
        work = torch.stack(out, axis)
    return work.reshape(shape)


# ------------------------------------------------------------------------- int8 lanes


def quantize_rows_int8(x: torch.Tensor, rotation: int = 256) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-token int8 of the rotated rows: `int8_linear.quantize_rows`
    (`internal/int8_linear.py:422-428`) for `rotation=256`:
    r = H256(x.float()) · (1/16); s = max(amax|r| / 127, 1e-12); q = clamp(rne(r / s), ±127).

    Build laws: `rotation=0` is the rotation-off lane (r = x.float()); `rotation=128` keeps the
    unnormalized H128 sums r, quantizes them with s as above, then returns the row scale
    s · fp32(1/√128), so codes never depend on the irrational constant.
    Returns int8 `[M, K]` and float32 `[M, 1]`."""
    flat = x.reshape(-1, x.shape[-1]).float()
    if rotation == 0:
        rotated = flat.clone()
    elif rotation == 128:
        rotated = hadamard(flat, 128)
    else:
        rotated = hadamard(flat, rotation).mul_(1.0 / math.isqrt(rotation))
    row_scale = (rotated.abs().amax(-1, keepdim=True) / 127.0).clamp_(min=SCALE_FLOOR)
    quantized = torch.round(rotated / row_scale).clamp_(-127, 127).to(torch.int8)
    if rotation == 128:
        row_scale = row_scale * torch.tensor(1.0 / math.sqrt(128.0), dtype=torch.float32)
    return quantized, row_scale


def int8_weight_rowwise(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-row int8 weight: `s = max(amax/127, 1e-12)`, `q = clamp(rne(w/s), ±127)`
    (`internal/probe.py:764-767`). Returns int8 `[N, K]`, float32 `[N]`."""
    w = w.float()
    scale = (w.abs().amax(dim=-1) / 127.0).clamp(min=SCALE_FLOOR)
    payload = torch.round(w / scale.unsqueeze(-1)).clamp(-127, 127)
    return payload.to(torch.int8), scale


def int8_weight_rotated(w: torch.Tensor, rotation: int) -> tuple[torch.Tensor, torch.Tensor]:
    """The weight side of a rotated int8 lane: each row rotated by the same orthonormal block
    Hadamard as the activations, then per-row int8 (`quantize_rows_int8`'s law on W's rows), so
    (H x)·(H w)ᵀ / n = x·wᵀ. The reference produces these bytes in tensorfs
    (`derive/microscale.py:117-138`, parity unpinned there); this is the build's producer."""
    q, s = quantize_rows_int8(w, rotation)
    return q, s.reshape(-1)


def int32_gemm(q: torch.Tensor, data: torch.Tensor, literal: bool = False) -> torch.Tensor:
    """`q.int32 @ data.int32ᵀ` (`internal/int8_linear.py:446`), exact. Evaluated as a float64
    matmul, which is exact while K·127² < 2**53, and checked against numpy int64 in the tests;
    `literal=True` runs the reference's own int32 matmul (the timed CPU baseline)."""
    if literal:
        return q.to(torch.int32) @ data.to(torch.int32).t()
    k = int(q.shape[-1])
    assert k * 127 * 127 < 2**53
    return (q.double() @ data.double().t()).to(torch.int32)


def int8_epilogue(
    acc: torch.Tensor, row_scale: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None,
    out_dtype: torch.dtype,
) -> torch.Tensor:
    """The int8 lane's float sequence after the exact int32 product: `acc.float()` (rounds
    past 2**24), `· row_scale` then `· w_scale` in float32, one cast to the output dtype
    (`internal/int8_linear.py:447-448`), then `+ bias` in that dtype (`:276`)."""
    out = acc.float().mul_(row_scale.reshape(-1, 1)).mul_(scale.float().reshape(1, -1))
    out = out.to(out_dtype)
    return out if bias is None else out + bias.to(out.dtype)


def int8_product(
    q: torch.Tensor, row_scale: torch.Tensor, data: torch.Tensor, scale: torch.Tensor,
    out_dtype: torch.dtype, literal: bool = False,
) -> torch.Tensor:
    """`_product`'s CPU branch (`internal/int8_linear.py:431-448`): int32 accumulate, then
    `(acc.float() · row_scale) · w_scale` in float32 (two roundings), then one cast."""
    return int8_epilogue(int32_gemm(q, data, literal), row_scale, scale, None, out_dtype)


def gelu_tanh(y: torch.Tensor) -> torch.Tensor:
    """tanh-GELU in float32 with the reference's constants (`internal/prebuilt.py:775`):
    0.5·y·(1 + tanh(0.79788456·(y + 0.044715·y³)))."""
    y = y.float()
    return 0.5 * y * (1.0 + torch.tanh(0.79788456 * (y + 0.044715 * y * y * y)))


def int8_linear(
    x: torch.Tensor, data: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None,
    out_dtype: torch.dtype, rotation: int = 256, gelu: bool = False, literal: bool = False,
) -> torch.Tensor:
    """The eager int8 linear (`internal/int8_linear.py:275-276,415-419`): quantize, product,
    then `+ bias` in the output dtype. `gelu=True` (build law for the DiT FFN-up epilogue)
    applies `gelu_tanh` to that result in float32 and casts once more. `literal=True` runs the
    reference's int32 matmul (the CPU path timed as the baseline)."""
    q, row_scale = quantize_rows_int8(x, rotation)
    out = int8_epilogue(int32_gemm(q, data, literal), row_scale, scale, bias, out_dtype)
    if gelu:
        out = gelu_tanh(out).to(out_dtype)
    return out.reshape(*x.shape[:-1], -1)


def int8_exact(
    x: torch.Tensor, data: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None,
    rotation: int = 256, gelu: bool = False,
) -> torch.Tensor:
    """The same product in float64 after quantization (`internal/prebuilt.py:751-763`'s role):
    what a kernel computes before its output rounding."""
    q, row_scale = quantize_rows_int8(x, rotation)
    out = int32_gemm(q, data).double() * row_scale.double() * scale.double().reshape(1, -1)
    if bias is not None:
        out = out + bias.double()
    if gelu:
        out = gelu_tanh(out.float()).double()
    return out


# ------------------------------------------------------------------------- fp8 rowwise


def fp8_quantize(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """`fp8_linear.eager_quantize` (`internal/fp8_linear.py:56-63`): per row
    s = max(float(amax|x|) / 448, 1e-12); q = e4m3(clamp(x.float() / s, ±448)), round to
    nearest even, e4m3 subnormals kept. Returns e4m3 `[M, K]` and float32 `[M, 1]`."""
    flat = x.reshape(-1, x.shape[-1])
    scale = (flat.abs().amax(dim=-1, keepdim=True).float() / E4M3_MAX).clamp(min=SCALE_FLOOR)
    q = (flat.float() / scale).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return q, scale


#: The producer prologue's codes (`internal/int8_linear.py:302-305`, `kernels/csrc/gemm/int8.h:25-26`).
NORM_LAYER, NORM_RMS = 1, 2
ACT_GELU, ACT_GELU_TANH, ACT_SITU, ACT_SWIGLU = 1, 2, 3, 4


def prologue(
    x: torch.Tensor, *, scale: torch.Tensor | None = None, shift: torch.Tensor | None = None,
    norm: int = 0, eps: float = 0.0, activation: int = 0, up: torch.Tensor | None = None,
) -> torch.Tensor:
    """The producer's prologue folded into the quantize pass, in float32 and in the reference
    kernel's order of operations (`kernels/csrc/gemm/rotate.cu:195-282`, contract
    `int8.h:25-47`): activation(norm(x)·(1 + scale[e]) + shift[e]), e = row // (rows // entries).
    - norm: mean = Σx/K (layer; 0 for RMS), rstd = rsqrt(Σ(x − mean)²/K + eps), (x − mean)·rstd.
    - activation 1: 0.5·y·(1 + erf(y·0.70710678)); 2: 0.5·y·(1 + tanh(0.79788456·(y + 0.044715·y³))).
    - 3 (SiTU, x = [hidden | gate]): (4·tanh(g/4) / (1 + e^-g))·(25·tanh(h/25)).
    - 4 (SwiGLU): silu(g) = g / (1 + e^-g) rounded to x's dtype, times up, rounded again; gate
      rows in x and up rows in `up`, or x = [up | gate] without `up`.
    Returns the float32 rows the rotation / quantization takes."""
    dtype = x.dtype
    flat = x.reshape(-1, x.shape[-1]).float()
    if activation == ACT_SITU:
        h, g = flat.chunk(2, -1)
        return (4.0 * torch.tanh(g * 0.25) / (1.0 + torch.exp(-g))) * (25.0 * torch.tanh(h / 25.0))
    if activation == ACT_SWIGLU:
        if up is None:
            u, g = flat.chunk(2, -1)
        else:
            g, u = flat, up.reshape(-1, up.shape[-1]).float()
        silu = (g / (1.0 + torch.exp(-g))).to(dtype).float()
        return (silu * u).to(dtype).float()
    v = flat
    if norm:
        k = float(v.shape[-1])
        mean = v.sum(-1, keepdim=True) / k if norm == NORM_LAYER else torch.zeros_like(v[:, :1])
        d = v - mean
        rstd = torch.rsqrt((d * d).sum(-1, keepdim=True) / k + eps)
        v = (v - mean) * rstd
    rows = v.shape[0]
    for table, kind in ((scale, "scale"), (shift, "shift")):
        if table is None:
            continue
        t = table.reshape(-1, v.shape[-1]).float()
        entry = torch.arange(rows) // (rows // t.shape[0])
        v = v * (1.0 + t[entry]) if kind == "scale" else v + t[entry]
    if activation == ACT_GELU:
        v = 0.5 * v * (1.0 + torch.erf(v * 0.70710678))
    elif activation == ACT_GELU_TANH:
        v = 0.5 * v * (1.0 + torch.tanh(0.79788456 * (v + 0.044715 * v * v * v)))
    return v


#: comfy-kitchen's frozen 16-level Lloyd-Max codebook, the one the reference's w4a8 producer
#: writes (`internal/prebuilt.py:679-682`).
W4A8_CODEBOOK = (
    -0.980602, -0.794529, -0.638165, -0.500986, -0.377321, -0.263187, -0.155210, -0.050720,
    0.052541, 0.156985, 0.265284, 0.379533, 0.502636, 0.638953, 0.794876, 0.980671,
)  # fmt: skip


def w4a8_unpack(codes: torch.Tensor, group_scale: torch.Tensor,
                codebook: torch.Tensor | None) -> torch.Tensor:  # fmt: skip
    """The int8 levels [N, K] of `w4a8.convrot` codes (`internal/prebuilt.py:471-492`):
    `codes` bytes [N, K/2], even k in the low nibble; `group_scale` E4M3 [N, K/16];
    level = clamp(round_half_even(codebook[q] · e4m3(group_scale)), ±127), one float32 multiply,
    a NaN product 0; `codebook` None is the uniform grid q − 8."""
    codes = codes.view(torch.uint8)
    rows, half = codes.shape
    levels = (torch.arange(-8, 8, dtype=torch.float32) if codebook is None
              else codebook.reshape(16).float())  # fmt: skip
    q = torch.stack((codes & 15, codes >> 4), dim=-1).reshape(rows, -1).long()
    grouped = levels[q].view(rows, -1, 16) * group_scale.float().unsqueeze(-1)
    return torch.round(grouped).nan_to_num_(0.0).clamp_(-127, 127).view(rows, -1).to(torch.int8)


def fp8_weight(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-row E4M3 weight (`internal/probe.py:706-709`)."""
    w = w.float()
    scale = (w.abs().amax(dim=-1) / E4M3_MAX).clamp(min=SCALE_FLOOR)
    payload = (w / scale.unsqueeze(-1)).clamp(-E4M3_MAX, E4M3_MAX)
    return payload.to(torch.float8_e4m3fn), scale


def fp8_exact(
    x: torch.Tensor, data: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None
) -> torch.Tensor:
    """`(q·Wᵀ)·s_x·s_w + bias` (`internal/fp8_linear.py:97-111`, `_scaled_mm` semantics) in
    float64 from the law's codes: e4m3 products and their sums are exact in float64 here."""
    q, sx = fp8_quantize(x)
    out = (q.double() @ data.double().t()) * sx.double() * scale.double().reshape(1, -1)
    return out if bias is None else out + bias.double()


def fp8_linear(
    x: torch.Tensor, data: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None,
    out_dtype: torch.dtype,
) -> torch.Tensor:
    """The CPU path timed as the fp8 baseline: `eager_quantize`, then dequantize and a float32
    matmul, both scales, one cast, then `+ bias` in the output dtype. The reference's own CPU
    call (`torch._scaled_mm` with row-wise scales) does not run on CPU torch 2.10, so this
    dequantize form stands in for it."""
    q, sx = fp8_quantize(x)
    out = (q.float() @ data.float().t()).mul_(sx).mul_(scale.float().reshape(1, -1))
    out = out.to(out_dtype)
    return out if bias is None else out + bias.to(out_dtype)


# ----------------------------------------------------------------------------- MXFP8


def e8m0_multipliers(byte: torch.Tensor) -> torch.Tensor:
    """E8M0 bytes → float32 by bit construction (`internal/encoding/formats.py:577-585`):
    b ↦ bits b<<23; 0 ↦ 2**-127 (bits 1<<22); 255 ↦ NaN."""
    raw = byte.view(torch.uint8)
    bits = raw.to(torch.int32) << 23
    bits = torch.where(raw == 0, torch.full_like(bits, 1 << 22), bits)
    mult = bits.view(torch.float32)
    return torch.where(raw == 255, torch.full_like(mult, float("nan")), mult)


def mx_quantize(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """`leaves.quantize_activation_mx` (`internal/encoding/leaves.py:1411-1424`): per 32-block,
    e = ceil(log2(amax/448)) (−127 for an all-zero block); byte = clamp(e+127, 0, 254);
    payload = e4m3(clamp(x / 2**(byte−127), ±448)). K % 32 == 0. Returns e4m3 `[M, K]` and
    uint8 `[M, K/32]`."""
    flat = x.reshape(-1, x.shape[-1])
    rows, cols = int(flat.shape[0]), int(flat.shape[1])
    work = flat.float().view(rows, cols // MX_BLOCK, MX_BLOCK)
    amax = work.abs().amax(dim=-1)
    exponent = torch.where(
        amax > 0, torch.ceil(torch.log2(amax / E4M3_MAX)), torch.full_like(amax, -127.0)
    )
    byte = (exponent + 127).clamp(0.0, 254.0).to(torch.uint8)
    payload = (work / e8m0_multipliers(byte).unsqueeze(-1)).view(rows, cols)
    return payload.clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn), byte


def mx_dequantize(payload: torch.Tensor, byte: torch.Tensor) -> torch.Tensor:
    """`MicroScaledDequant.decode`'s value (`internal/encoding/formats.py:638-650`) in float32,
    for a row-major grid `[rows, ceil(K/32)]`: exact."""
    rows, cols = int(payload.shape[0]), int(payload.shape[1])
    mult = e8m0_multipliers(byte.contiguous())
    return payload.float() * mult.repeat_interleave(MX_BLOCK, dim=1)[:, :cols]


def mx_exact(
    x: torch.Tensor, data: torch.Tensor, wbyte: torch.Tensor, bias: torch.Tensor | None
) -> torch.Tensor:
    """`_scaled_mm` with 1×32 E8M0 block scales (`internal/encoding/leaves.py:1509-1519`) in
    float64 from the law's codes: Σ_k (p_x·2^e_x)(p_w·2^e_w) + bias."""
    p, b = mx_quantize(x)
    out = mx_dequantize(p, b).double() @ mx_dequantize(data, wbyte).double().t()
    return out if bias is None else out + bias.double()


def mx_linear(
    x: torch.Tensor, data: torch.Tensor, wbyte: torch.Tensor, bias: torch.Tensor | None,
    out_dtype: torch.dtype,
) -> torch.Tensor:
    """The CPU path timed as the MXFP8 baseline: `quantize_activation_mx`, exact E8M0 dequant
    of both operands, a float32 matmul, one cast, then `+ bias` in the output dtype."""
    p, b = mx_quantize(x)
    out = (mx_dequantize(p, b) @ mx_dequantize(data, wbyte).t()).to(out_dtype)
    return out if bias is None else out + bias.to(out_dtype)


def _blocked_shape(rows: int, cols: int) -> tuple[int, int]:
    return -(-rows // 128) * 128, -(-cols // 4) * 4


def to_blocked(scales: torch.Tensor) -> torch.Tensor:
    """Row-major `[rows, cols]` scale bytes → cuBLAS's 128×4 tiled layout
    (`internal/encoding/formats.py:158-170`)."""
    rows, cols = int(scales.shape[0]), int(scales.shape[1])
    prow, pcol = _blocked_shape(rows, cols)
    padded = torch.zeros(prow, pcol, dtype=scales.dtype)
    padded[:rows, :cols] = scales
    tiles = padded.view(prow // 128, 128, pcol // 4, 4).permute(0, 2, 1, 3)
    return tiles.reshape(-1, 4, 32, 4).transpose(1, 2).reshape(-1).contiguous()


def from_blocked(blocked: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    """`to_blocked`'s inverse (`internal/encoding/formats.py:173-178`)."""
    prow, pcol = _blocked_shape(rows, cols)
    tiles = blocked.reshape(-1, 32, 4, 4).transpose(1, 2).reshape(prow // 128, pcol // 4, 128, 4)
    return tiles.permute(0, 2, 1, 3).reshape(prow, pcol)[:rows, :cols]


# ------------------------------------------------------------- W4A4 int4-g64 SVDQuant


def int4_quantize(v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Build law (no reference counterpart; the reference's W4A4 is nvfp4,
    `internal/svdq_linear.py:605-618`): per row and per 64-group of float32 values v,
    s = fp16(amax|v| / 7); q = 0 where s == 0, else clamp(rne(v / float(s)), −8, 7).
    Returns int8 codes `[M, K]` (values −8..7) and float16 scales `[M, K/64]`."""
    rows, cols = int(v.shape[0]), int(v.shape[1])
    work = v.float().reshape(rows, cols // INT4_GROUP, INT4_GROUP)
    s16 = (work.abs().amax(dim=-1) / INT4_MAX).to(torch.float16)
    s32 = s16.float().unsqueeze(-1)
    q = torch.round(work / s32).clamp(-8, 7)
    q = torch.where(s32 == 0, torch.zeros_like(q), q)
    return q.to(torch.int8).reshape(rows, cols), s16


def pack_int4(q: torch.Tensor) -> torch.Tensor:
    """Codes −8..7 `[R, C]` → bytes `[R, C/2]`, element 2k in the low nibble (the reference's
    nibble order, `internal/svdq_linear.py:482-484`)."""
    u = (q.to(torch.int16) & 0xF).to(torch.uint8)
    return (u[:, 0::2] | (u[:, 1::2] << 4)).contiguous()


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    """`pack_int4`'s inverse: signed codes as int8."""
    lo = (packed & 0xF).to(torch.int16)
    hi = (packed >> 4).to(torch.int16)
    both = torch.stack((lo, hi), dim=-1).reshape(packed.shape[0], -1)
    return torch.where(both >= 8, both - 16, both).to(torch.int8)


def svdq_smooth(x: torch.Tensor, p: torch.Tensor) -> torch.Tensor:
    """`bf16(x · p)` as float32 (`internal/svdq_linear.py:592-595`)."""
    flat = x.reshape(-1, int(p.numel()))
    return (flat.float() * p.float()).to(torch.bfloat16).float()


def svdq_down(x: torch.Tensor, down: torch.Tensor) -> torch.Tensor:
    """The low-rank branch's input `bf16(x · downᵀ)`, down `[R, K]` (`internal/svdq_linear.py:
    598-602`): x in its half dtype (bf16 for float32 x) and down cast to that dtype, the
    products summed exactly (float64 here; the reference accumulates in float32), one
    rounding to bf16."""
    flat = x.reshape(-1, int(down.shape[1]))
    half = flat.dtype if flat.dtype in (torch.bfloat16, torch.float16) else torch.bfloat16
    return (flat.to(half).double() @ down.to(half).double().t()).to(torch.bfloat16)


def svdq_weight(
    w: torch.Tensor, p: torch.Tensor, down: torch.Tensor, up: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    """Build weight producer (the reference's is tensorfs's SVDQ writer, not in the repository):
    the residual W − up·down moved into the smoothed basis (÷ p per input channel, so
    (x·p)·Rᵀ = x·(W − up·down)ᵀ), then `int4_quantize` per 64-group. down `[R, K]`, up `[N, R]`.
    Returns packed codes `[N, K/2]` and float16 scales `[N, K/64]`."""
    residual = w.double() - up.double() @ down.double()
    smoothed = (residual / p.double().reshape(1, -1)).float()
    q, s = int4_quantize(smoothed)
    return pack_int4(q), s


def svdq_exact(
    x: torch.Tensor, p: torch.Tensor, wcodes: torch.Tensor, wscale: torch.Tensor,
    down: torch.Tensor, up: torch.Tensor, bias: torch.Tensor | None,
) -> torch.Tensor:
    """The W4A4 product in float64 (`internal/svdq_linear.py:639-659`'s structure with the
    int4-g64 law): Σ_g (Σ_{k∈g} qx·qw)·sx[m,g]·sw[n,g] + bf16(x·downᵀ)·upᵀ + bias."""
    qx, sx = int4_quantize(svdq_smooth(x, p))
    qw = unpack_int4(wcodes)
    rows, cols = int(qx.shape[0]), int(qx.shape[1])
    groups = cols // INT4_GROUP
    ax = qx.double().reshape(rows, groups, INT4_GROUP) * sx.double().unsqueeze(-1)
    aw = qw.double().reshape(-1, groups, INT4_GROUP) * wscale.double().unsqueeze(-1)
    out = ax.reshape(rows, cols) @ aw.reshape(-1, cols).t()
    out = out + svdq_down(x, down).double() @ up.double().t()
    return out if bias is None else out + bias.double()


def svdq_linear(
    x: torch.Tensor, p: torch.Tensor, wcodes: torch.Tensor, wscale: torch.Tensor,
    down: torch.Tensor, up: torch.Tensor, bias: torch.Tensor | None, out_dtype: torch.dtype,
) -> torch.Tensor:
    """The CPU path timed as the W4A4 baseline (`internal/svdq_linear.py:639-659` with the
    int4-g64 law): activations quantized, both operands dequantized to float32, one float32
    matmul, plus the bf16 low-rank branch and the bias in float32, one cast."""
    qx, sx = int4_quantize(svdq_smooth(x, p))
    rows, cols = int(qx.shape[0]), int(qx.shape[1])
    groups = cols // INT4_GROUP
    ax = (qx.float().reshape(rows, groups, INT4_GROUP) * sx.float().unsqueeze(-1)).reshape(rows, cols)
    qw = unpack_int4(wcodes)
    aw = (qw.float().reshape(-1, groups, INT4_GROUP) * wscale.float().unsqueeze(-1)).reshape(-1, cols)
    out = ax @ aw.t() + svdq_down(x, down).float() @ up.float().t()
    if bias is not None:
        out = out + bias.float()
    return out.to(out_dtype)


# ------------------------------------------------------------ W4A4 svdq.nvfp4 SVDQuant

#: svdq.nvfp4's second-level bound (E4M3 max · E2M1 max), the block-scale floor (E4M3's least
#: subnormal) and the activation scale's floor (`internal/svdq_linear.py:44-47`, `:590`).
SVDQ_LEVELS_MAX = 448.0 * 6.0
SVDQ_BLOCK_FLOOR = 2.0**-9
SVDQ_INPUT_FLOOR = 1e-30
#: The E2M1 thresholds of `quantize` (`internal/svdq_linear.py:613-616`): (bound, inclusive).
SVDQ_THRESHOLDS = ((0.25, False), (0.75, True), (1.25, False), (1.75, True), (2.5, False),
                   (3.5, True), (5.0, False))  # fmt: skip


def svdq_nvfp4_input_scale(x: torch.Tensor, p: torch.Tensor,
                           stored: torch.Tensor | None = None) -> torch.Tensor:
    """`activation_scale` (`internal/svdq_linear.py:582-590`): the stored `input_scale`, else
    `max_j(max_i |x_ij| · p_j) / 2688` in float32, floored at 1e-30. Returns float32 [1]."""
    if stored is not None:
        return stored.float().reshape(1)
    flat = x.reshape(-1, int(p.numel()))
    amax = (flat.abs().amax(0).float() * p.float()).amax()
    return (amax / SVDQ_LEVELS_MAX).clamp(min=SVDQ_INPUT_FLOOR).reshape(1)


def svdq_nvfp4_quantize(xs: torch.Tensor, g: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """`quantize` (`internal/svdq_linear.py:605-618`): `xs` float32 [M, K] (already bf16(x·p))
    at second level g → E2M1 codes [M, K] (u8, sign in bit 3) and E4M3 scales [M, K/16]:
    scale = e4m3(clamp(amax / (6g), 2^-9, 448)), code = the threshold count of |xs/(scale·g)|
    (+8 where xs < 0)."""
    rows, cols = int(xs.shape[0]), int(xs.shape[1])
    blocks = xs.float().view(rows, cols // NVFP4_BLOCK, NVFP4_BLOCK)
    gv = g.float().reshape(())
    amax = blocks.abs().amax(-1)
    scale = (amax / (6.0 * gv)).clamp(SVDQ_BLOCK_FLOOR, E4M3_MAX).to(torch.float8_e4m3fn)
    a = (blocks / (scale.float() * gv).unsqueeze(-1)).abs()
    code = torch.zeros_like(blocks, dtype=torch.uint8)
    for bound, inclusive in SVDQ_THRESHOLDS:
        code = code + ((a >= bound) if inclusive else (a > bound)).to(torch.uint8)
    code = code + (blocks < 0).to(torch.uint8) * 8
    return code.view(rows, cols), scale


def svdq_nvfp4_pack(codes: torch.Tensor) -> torch.Tensor:
    """E2M1 codes [M, K] → bytes [M, K/2], element 2k in the low nibble (the stored order the
    kernels read, `internal/svdq_linear.py:520`)."""
    return (codes[:, 0::2] | (codes[:, 1::2] << 4)).contiguous()


def svdq_nvfp4_values(codes: torch.Tensor, scales: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
    """`_values` (`internal/svdq_linear.py:627-632`): codes [R, C] (u8) with E4M3 scales [R, C/16]
    → float32 `(E2M1 · scale) · g`."""
    lut = torch.tensor(E2M1_VALUES, dtype=torch.float32)
    blocks = lut[codes.long()].view(codes.shape[0], -1, NVFP4_BLOCK)
    return (blocks * scales.float().unsqueeze(-1) * g.float().reshape(())).view(codes.shape)


def _svdq_weight_values(roles: dict) -> torch.Tensor:
    packed = roles["weight"].view(torch.uint8)
    codes = torch.stack((packed & 0x0F, packed >> 4), dim=-1).view(packed.shape[0], -1)
    return svdq_nvfp4_values(codes, roles["scale"], roles["scale_2"])


def svdq_nvfp4_exact(x: torch.Tensor, roles: dict, bias: torch.Tensor | None) -> torch.Tensor:
    """The svdq.nvfp4 linear in float64 from the law's codes (`internal/svdq_linear.py:427-438`,
    the reference's own probe target): `(values(q(x·p)) · values(W)ᵀ) · c + bf16(x·downᵀ) · upᵀ
    + bias`, every product and sum exact."""
    p = roles["pre_quant_scale"]
    g = svdq_nvfp4_input_scale(x, p, roles.get("input_scale"))
    codes, scales = svdq_nvfp4_quantize(svdq_smooth(x, p), g)
    out = svdq_nvfp4_values(codes, scales, g).double() @ _svdq_weight_values(roles).double().t()
    if roles.get("channel_scale") is not None:
        out = out * roles["channel_scale"].double().reshape(1, -1)
    out = out + svdq_down(x, roles["lowrank_down"]).double() @ roles["lowrank_up"].double().t()
    return out if bias is None else out + bias.double()


def svdq_nvfp4_eager(x: torch.Tensor, roles: dict, bias: torch.Tensor | None,
                     out_dtype: torch.dtype) -> torch.Tensor:
    """`eager` (`internal/svdq_linear.py:639-659`), the CPU path timed as the svdq.nvfp4
    baseline: the activation fake-quantized, float32 matmul against the decoded weight, `· c`,
    `+` the low-rank branch and the bias in float32, one cast."""
    p = roles["pre_quant_scale"]
    flat = x.reshape(-1, int(p.numel()))
    g = svdq_nvfp4_input_scale(flat, p, roles.get("input_scale"))
    codes, scales = svdq_nvfp4_quantize(svdq_smooth(flat, p), g)
    y = svdq_nvfp4_values(codes, scales, g) @ _svdq_weight_values(roles).t()
    if roles.get("channel_scale") is not None:
        y = y * roles["channel_scale"].float()
    half = flat.dtype if flat.dtype in (torch.bfloat16, torch.float16) else torch.bfloat16
    down = (flat.to(half) @ roles["lowrank_down"].to(half).t()).to(torch.bfloat16)
    y = y + down.float() @ roles["lowrank_up"].float().t()
    if bias is not None:
        y = y + bias.float()
    return y.to(out_dtype)


# ------------------------------------------------------------------------ decode laws


def decode_int8_convrot(payload: torch.Tensor, scale: torch.Tensor, size: int,
                        dtype: torch.dtype) -> torch.Tensor:
    """`Int8ConvRotDequant.decode` (`internal/encoding/formats.py:733-752`):
    hadamard(int32 data)·scale·(1/√size) in float32, one cast."""
    block = hadamard(payload.to(torch.int32), size).to(torch.float32)
    block.mul_(scale.to(torch.float32).reshape(-1, 1)).mul_(1.0 / math.isqrt(size))
    return block.to(dtype)


def decode_rowwise(payload: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """`RowwiseDequant.decode` (`internal/encoding/formats.py:557-569`): data·scale[row] in
    float32, one cast."""
    rows = int(payload.shape[0])
    return (payload.to(torch.float32) * scale.to(torch.float32).reshape(rows, 1)).to(dtype)


def decode_columnwise(payload: torch.Tensor, scale: torch.Tensor,
                      dtype: torch.dtype) -> torch.Tensor:
    """`RowwiseDequant.decode` for a `.columnwise` scheme (`internal/encoding/formats.py:
    557-569`): data·scale[column] in float32, one cast."""
    cols = int(payload.shape[-1])
    return (payload.to(torch.float32) * scale.to(torch.float32).reshape(1, cols)).to(dtype)


def decode_tensorwise(payload: torch.Tensor, scale: torch.Tensor,
                      dtype: torch.dtype) -> torch.Tensor:
    """`TensorwiseDequant.decode` (`internal/encoding/formats.py:485-492`): data·scale in
    float32, one cast."""
    return (payload.to(torch.float32) * scale.to(torch.float32).reshape(())).to(dtype)


#: E2M1 by nibble, bit 3 the sign (`internal/encoding/formats.py:755-759`).
E2M1_VALUES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
               -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)  # fmt: skip
NVFP4_BLOCK = 16


def nvfp4_values(weight: torch.Tensor, scale: torch.Tensor, scale_2: torch.Tensor,
                 high_first: bool = False, divide: bool = False) -> torch.Tensor:
    """`formats.nvfp4_values` (`internal/encoding/formats.py:762-783`) for one matrix: bytes
    `[R, C/2]` (element 2k in the low nibble, or the high one with `high_first`), a row-major
    E4M3 grid `[R, C/16]`, a float32 `scale_2` → float32 `[R, C]`: `(e2m1·s)·g`, or
    `e2m1·(s/g)` with `divide`."""
    rows, cols = int(weight.shape[0]), int(weight.shape[1]) * 2
    w = weight.view(torch.uint8)
    pair = (w >> 4, w & 0x0F) if high_first else (w & 0x0F, w >> 4)
    codes = torch.stack(pair, dim=-1).reshape(rows, cols)
    lut = torch.tensor(E2M1_VALUES, dtype=torch.float32)
    blocks = lut[codes.long()].view(rows, cols // NVFP4_BLOCK, NVFP4_BLOCK)
    second = scale_2.to(torch.float32).reshape(())
    block_scale = scale.to(torch.float32).reshape(rows, cols // NVFP4_BLOCK, 1)
    if divide:
        return blocks.mul_(block_scale / second).view(rows, cols)
    blocks.mul_(block_scale)
    return blocks.view(rows, cols).mul_(second)


def decode_nvfp4(weight: torch.Tensor, scale: torch.Tensor, scale_2: torch.Tensor, layout: str,
                 high_first: bool, divide: bool, post: torch.Tensor | None,
                 dtype: torch.dtype) -> torch.Tensor:
    """The nvfp4 decode of one matrix (`internal/decode_schemes.py:362-402`,
    `internal/decode_cores.py:196-230`): `nvfp4_values`, then `· post[j]` (AWQ's
    `pre_quant_scale`) when given, one cast. `scale` row-major or in cuBLAS's 128x4 tiles."""
    rows, cols = int(weight.shape[0]), int(weight.shape[1]) * 2
    grid = from_blocked(scale.reshape(-1), rows, cols // NVFP4_BLOCK) \
        if layout == "cublas_128x4" else scale.reshape(rows, cols // NVFP4_BLOCK)
    value = nvfp4_values(weight, grid, scale_2, high_first, divide)
    if post is not None:
        factor = post.reshape(-1).to(torch.float32)
        value = value * (factor if factor.numel() == cols else factor[0])
    return value.to(dtype)


def decode_svdq_nvfp4(weight: torch.Tensor, scale: torch.Tensor, scale_2: torch.Tensor,
                      layout: str, high_first: bool, divide: bool,
                      channel: torch.Tensor | None, smooth: torch.Tensor, down: torch.Tensor,
                      up: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """The svdq.nvfp4 decode (`internal/decode_schemes.py:464-489`): the nvfp4 value,
    `· channel[i]`, `· smooth[j]`, then `+ up[i, r]·down[r, j]` for r in order, each product
    rounded to float32 before its add; one cast."""
    rows, cols = int(weight.shape[0]), int(weight.shape[1]) * 2
    value = decode_nvfp4(weight, scale, scale_2, layout, high_first, divide, None, torch.float32)
    if channel is not None:
        value = value * channel.to(torch.float32).reshape(rows, 1)
    value = value * smooth.to(torch.float32).reshape(1, cols)
    u = up.to(torch.float32).reshape(rows, -1)
    d = down.to(torch.float32).reshape(u.shape[1], cols)
    for r in range(u.shape[1]):
        value.add_(torch.mul(u[:, r : r + 1], d[r : r + 1, :]))
    return value.to(dtype)


def decode_mxfp8(payload: torch.Tensor, scale: torch.Tensor, layout: str,
                 dtype: torch.dtype) -> torch.Tensor:
    """`MicroScaledDequant.decode` (`internal/encoding/formats.py:638-650`) for one matrix."""
    rows, cols = int(payload.shape[0]), int(payload.shape[1])
    blocks = -(-cols // MX_BLOCK)
    grid = from_blocked(scale.reshape(-1), rows, blocks) if layout == "cublas_128x4" \
        else scale.reshape(rows, blocks)
    return mx_dequantize(payload, grid).to(dtype)


# -------------------------------------------------------------------- weight encoders
# Build laws: the reference's producers live in tensorfs (derive/microscale.py:117-408), whose
# arithmetic is not in the reference, so these encoders are this build's own. int8.convrot and
# fp8.rowwise weights use `int8_weight_rotated` and `fp8_weight` above; mxfp8 uses `mx_quantize`.


def e2m1_code(r: torch.Tensor) -> torch.Tensor:
    """float32 → E2M1 nibble, nearest even on ties, |r| > 6 saturating to 6; bit 3 set where
    r < 0 (build law)."""
    a = r.abs()
    m = torch.full_like(a, 7, dtype=torch.int32)
    for bound, code, inclusive in ((5.0, 6, True), (3.5, 5, False), (2.5, 4, True), (1.75, 3, False),
                                   (1.25, 2, True), (0.75, 1, False), (0.25, 0, True)):  # fmt: skip
        m = torch.where(a <= bound if inclusive else a < bound, torch.full_like(m, code), m)
    return m | torch.where(r < 0, 8, 0).to(torch.int32)


def encode_nvfp4(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, int]:
    """nvfp4 producer (build law; the reference's is tensorfs's `nvfp4-min-sse/1`,
    `derive/microscale.py:146-217`): g = amax|w| / (448·6) (1 for an all-zero matrix); per
    16-block the E4M3 scale among c0 = e4m3(amax_b / (6g)), c0 − 1 and c0 + 1 (positive codes,
    first of equals in that order) whose decode `(e2m1·s)·g` has the least float32 squared error
    summed in k order; codes e2m1 of w / (s·g). Returns bytes [R, K/2] (low nibble first), E4M3
    bytes [R, K/16], g (float32 scalar) and the count of |w/(s·g)| > 6."""
    x = w.float()
    rows, cols = x.shape
    blocks = x.reshape(rows, cols // 16, 16)
    amax_t = x.abs().max() if x.numel() else torch.tensor(0.0)
    g = (amax_t / torch.tensor(E4M3_MAX * 6.0)) if amax_t > 0 else torch.tensor(1.0)
    amax_b = blocks.abs().amax(dim=-1)
    six_g = torch.tensor(6.0) * g
    c0 = (amax_b / six_g).clamp(max=E4M3_MAX).to(torch.float8_e4m3fn).view(torch.uint8).to(torch.int32)
    cands = (c0, torch.where(c0 > 1, c0 - 1, c0), torch.where(c0 < 0x7E, c0 + 1, c0))
    lut = torch.tensor(E2M1_VALUES, dtype=torch.float32)

    def trial(code: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        s = code.to(torch.uint8).view(torch.float8_e4m3fn).float().unsqueeze(-1)
        d = s * g
        r = torch.where(d > 0, blocks / torch.where(d > 0, d, torch.ones_like(d)), torch.zeros_like(blocks))
        q = e2m1_code(r)
        value = torch.where(d > 0, (lut[q.long()] * s) * g, torch.zeros_like(blocks))
        diff = blocks - value
        err = torch.zeros_like(amax_b)
        for k in range(16):
            err = err + diff[..., k] * diff[..., k]
        return err, q, r

    best = c0.clone()
    best_err = torch.full_like(amax_b, float("inf"))
    for code in cands:
        err, _, _ = trial(code)
        take = err < best_err
        best = torch.where(take, code, best)
        best_err = torch.where(take, err, best_err)
    _, q, r = trial(best)
    saturated = int((r.abs() > 6.0).sum())
    q = q.reshape(rows, cols).to(torch.uint8)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).contiguous()
    return packed, best.to(torch.uint8), g.reshape(()).float(), saturated


def encode_w4a8(w: torch.Tensor, codebook: torch.Tensor | None = None,
                ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """w4a8.convrot producer (build law; the reference's is tensorfs's
    `w4a8-convrot256-fixed/1`, `derive/microscale.py:349-408`): int8.convrot's rotated rows r
    and row scale s (`quantize_rows_int8`), t = r / s; per 16-group σ = e4m3(max|t| / max|c|)
    and each code the nearest of the levels clamp(rne(c[q]·σ), ±127) — the unpack law
    (`w4a8_unpack`) — first on a tie. Returns codes [N, K/2] (even k low), E4M3 [N, K/16] and
    the float32 row scale [N]."""
    cb = torch.tensor(W4A8_CODEBOOK, dtype=torch.float32) if codebook is None else codebook.float()
    x = w.float()
    rows, cols = x.shape
    r = hadamard(x, 256).mul_(1.0 / 16)
    s = (r.abs().amax(dim=-1) / 127.0).clamp(min=SCALE_FLOOR)
    t = (r / s.unsqueeze(-1)).view(rows, cols // 16, 16)
    ga = t.abs().amax(dim=-1)
    sb = (ga / cb.abs().max()).clamp(max=E4M3_MAX).to(torch.float8_e4m3fn)
    sigma = sb.float().unsqueeze(-1)
    levels = torch.round(cb.view(1, 1, 16) * sigma).nan_to_num_(0.0).clamp_(-127, 127)
    dist = (levels.unsqueeze(-2) - t.unsqueeze(-1)).abs()
    code = dist.argmin(dim=-1).to(torch.uint8).view(rows, cols)
    packed = (code[:, 0::2] | (code[:, 1::2] << 4)).contiguous()
    return packed, sb.view(torch.uint8), s


# ------------------------------------------------------------- independent bit laws


def e4m3_bits_numpy(v: np.ndarray) -> np.ndarray:
    """float32 → OCP E4M3FN byte by integer arithmetic only (round to nearest even, subnormals
    at 2**-9 steps, |v| > 448 → NaN 0x7F like an unsaturated cast). An independent encoder the
    tests hold torch's cast (`.to(torch.float8_e4m3fn)`) and the kernels' against."""
    bits = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32).astype(np.int64)
    sign = (bits >> 31) << 7
    mag = bits & 0x7FFFFFFF
    exp = mag >> 23
    man = mag & 0x7FFFFF
    out = np.zeros_like(mag)
    # normal e4m3: f32 exponent 121..135 (2**-6 .. 2**8); keep 3 mantissa bits
    e8 = exp - 127 + 7
    normal = e8 >= 1
    shift = np.where(normal, 20, 20 + (1 - e8))  # subnormal: fewer kept bits
    full = np.where(normal, man | 0x800000, man | 0x800000)
    shift = np.minimum(shift, 40)
    kept = full >> shift
    rem = full & ((np.int64(1) << shift) - 1)
    half = np.int64(1) << (shift - 1)
    up = (rem > half) | ((rem == half) & ((kept & 1) == 1))
    kept = kept + up
    # normal: kept holds 1.mmm (4 bits, maybe 5 after carry); value = kept·2**(e8-7-3)
    n_code = np.where(kept >= 16, ((e8 + 1) << 3) | ((kept >> 1) & 7), (e8 << 3) | (kept & 7))
    s_code = kept  # subnormal: kept counts 2**-9 units (carry into 8 gives the first normal)
    code = np.where(normal, n_code, s_code)
    zero = (mag == 0) | (exp < 127 - 7 - 3 - 1)  # below half the smallest subnormal
    code = np.where(zero, 0, code)
    nan = (exp == 255) | (code > 0x7E)
    code = np.where(nan, 0x7F, code)
    out = (sign | code).astype(np.uint8)
    return out

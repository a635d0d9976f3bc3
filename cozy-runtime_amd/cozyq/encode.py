"""Weight encoders on gfx950: cozyq's stand-ins for the producers cozy-runtime delegates to
tensorfs (`derive/microscale.py:146-408`: `encode_nvfp4`, `encode_fp8_rowwise`,
`encode_int8_convrot256`, `encode_w4a8`), plus `encode_mxfp8`.

Each takes a float32 / bf16 / fp16 matrix on the GPU and returns an `Encoded` with the
reference's fields: the payload and its companions (suffix, dtype, shape, bytes — here device
tensors rather than host bytes), and the measured acceptance facts `saturated`, `sse`, `energy`,
`max_abs_err` (`derive/microscale.py:64-110`), taken on the GPU by decoding the result with the
decode kernels and comparing it with the input (`cozyq_measure`). Refusals keep the reference's
`UnsupportedInput` messages. The arithmetic of each producer is this build's (the reference's is
in tensorfs); `include/cozyq.h` states each law and the oracle restates it.
"""

from __future__ import annotations

from typing import Any, NamedTuple

from cozyq import decode as dec

Tensor = Any

#: The rotation group and the fixed 16-level codebook of the w4a8 producer
#: (`derive/microscale.py:290,337-345`).
CONVROT_GROUP = 256
W4A8_GROUP = 16
W4A8_CODEBOOK = (
    -0.980602, -0.794529, -0.638165, -0.500986, -0.377321, -0.263187, -0.155210, -0.050720,
    0.052541, 0.156985, 0.265284, 0.379533, 0.502636, 0.638953, 0.794876, 0.980671,
)  # fmt: skip
NVFP4_BLOCK = 16
#: svdq.int4g64's K-group (this build's W4A4 variant).
SVDQ_INT4_GROUP = 64
MX_BLOCK = 32
E4M3_MAX = 448.0
#: float64 partials the measure folds through.
_PARTS = 1024


class UnsupportedInput(ValueError):
    """An input this family does not encode (`cozy_runtime.author.UnsupportedInput`)."""


class Companion(NamedTuple):
    """One scale sibling: suffix, header dtype, shape, and the stored bytes (a device tensor)."""

    suffix: str
    dtype: str
    shape: list[int]
    raw: Tensor


class Encoded(NamedTuple):
    payload_dtype: str
    payload_shape: list[int]
    payload: Tensor
    companions: list[Companion]
    saturated: int
    sse: float
    energy: float
    max_abs_err: float

    def relative_frobenius(self) -> float:
        """||W − dequant(quant(W))||_F / ||W||_F; 0 for an all-zero tensor."""
        return float((self.sse / self.energy) ** 0.5) if self.energy > 0 else 0.0


def _in_type(torch: Any, t: Tensor) -> int:
    return {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[t.dtype]


def _prepare(torch: Any, key: str, values: Tensor, block: int) -> tuple[Any, Tensor, int, int]:
    """`_require_2d` (`derive/microscale.py:113-128`) plus the device and dtype this build
    encodes from."""
    from cozyq.prebuilt import library

    if values.dim() != 2:
        raise UnsupportedInput(
            f"{key!r} is rank {values.dim()}: this family encodes 2-D GEMM weights, and a norm "
            "or a bias stays at source precision rather than being reshaped into one")  # fmt: skip
    rows, cols = int(values.shape[0]), int(values.shape[1])
    if cols % block:
        raise UnsupportedInput(
            f"{key!r} has {cols} columns, not a multiple of the {block}-element block — the "
            "encoding's blocking is a shape fact and padding it would change the tensor the "
            "consumer reads")  # fmt: skip
    if values.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise UnsupportedInput(f"{key!r} is {values.dtype}: the encoders read f32, bf16 or f16")
    if getattr(values.device, "type", None) != "cuda":
        raise ValueError(f"cozyq encodes on the GPU; {key!r} is on {values.device}")
    values = values.contiguous()
    if values.data_ptr() % 16:
        values = values.clone()
    if rows and not bool(torch.isfinite(values).all()):
        raise UnsupportedInput(f"{key!r} contains a non-finite weight — refuse, never encode")
    return library(values.device.index or 0), values, rows, cols


def _measured(torch: Any, ops: Any, values: Tensor, decoded: Tensor) -> tuple[float, float, float]:
    partial = torch.empty(_PARTS * 3, dtype=torch.float64, device=values.device)
    out = torch.empty(3, dtype=torch.float64, device=values.device)
    code = ops._lib.cozyq_measure(ops.index, values.data_ptr(), _in_type(torch, values),
                                  decoded.data_ptr(), values.numel(), partial.data_ptr(), _PARTS,
                                  out.data_ptr(), ops._stream())  # fmt: skip
    ops._check(code, "the encode measure")
    sse, energy, worst = (float(v) for v in out.cpu())
    return sse, energy, worst


def _decoded(torch: Any, scheme: str, params: dict, parts: dict, shape: tuple[int, int],
             device: Any) -> Tensor:
    out = torch.empty(shape, dtype=torch.float32, device=device)
    dec.decode(torch, scheme, params, parts, out)
    return out


def encode_int8_convrot256(torch: Any, key: str, values: Tensor) -> Encoded:
    """int8.convrot with 256-groups (`derive/microscale.py:295-334`): payload I8 [R, C] and
    `.weight_scale` F32 [R]."""
    ops, values, rows, cols = _prepare(torch, key, values, CONVROT_GROUP)
    q = torch.empty(rows, cols, dtype=torch.int8, device=values.device)
    scale = torch.empty(rows, dtype=torch.float32, device=values.device)
    if rows:
        code = ops._lib.cozyq_encode_int8_convrot(ops.index, values.data_ptr(),
                                                  _in_type(torch, values), q.data_ptr(),
                                                  scale.data_ptr(), rows, cols, ops._stream())  # fmt: skip
        ops._check(code, "the int8.convrot encoder")
    params = {"rotation": "kron_regular_h4", "rotation_size": CONVROT_GROUP}
    sse, energy, worst = (0.0, 0.0, 0.0) if not rows else _measured(
        torch, ops, values, _decoded(torch, "int8.convrot", params, {"weight": q, "scale": scale},
                                     (rows, cols), values.device))  # fmt: skip
    return Encoded("I8", [rows, cols], q, [Companion(".weight_scale", "F32", [rows], scale)], 0,
                   sse, energy, worst)  # fmt: skip


def encode_fp8_rowwise(torch: Any, key: str, values: Tensor) -> Encoded:
    """fp8.rowwise (`derive/microscale.py:223-262`): payload F8_E4M3 [R, C] and `.weight_scale`
    F32 [R]."""
    ops, values, rows, cols = _prepare(torch, key, values, 8)
    q = torch.empty(rows, cols, dtype=torch.float8_e4m3fn, device=values.device)
    scale = torch.empty(rows, dtype=torch.float32, device=values.device)
    if rows:
        code = ops._lib.cozyq_encode_fp8_rowwise(ops.index, values.data_ptr(),
                                                 _in_type(torch, values), q.data_ptr(),
                                                 scale.data_ptr(), rows, cols, ops._stream())  # fmt: skip
        ops._check(code, "the fp8.rowwise encoder")
    sse, energy, worst = (0.0, 0.0, 0.0) if not rows else _measured(
        torch, ops, values, _decoded(torch, "fp8.rowwise", {}, {"weight": q, "scale": scale},
                                     (rows, cols), values.device))  # fmt: skip
    return Encoded("F8_E4M3", [rows, cols], q,
                   [Companion(".weight_scale", "F32", [rows], scale)], 0, sse, energy, worst)  # fmt: skip


def encode_mxfp8(torch: Any, key: str, values: Tensor, scale_layout: str = "cublas_128x4") -> Encoded:
    """mxfp8 (`internal/encoding/formats.py:588-650`'s stored form): payload F8_E4M3 [R, C] and
    `.weight_scale` F8_E8M0 row-major [R, C/32] or in cuBLAS's 128x4 tiles."""
    ops, values, rows, cols = _prepare(torch, key, values, MX_BLOCK)
    tiled = scale_layout == "cublas_128x4"
    q = torch.empty(rows, cols, dtype=torch.float8_e4m3fn, device=values.device)
    shape = list(dec.blocked_shape(rows, cols // MX_BLOCK)) if tiled else [rows, cols // MX_BLOCK]
    scale = torch.zeros(shape, dtype=torch.uint8, device=values.device)
    if rows:
        code = ops._lib.cozyq_encode_mxfp8(ops.index, values.data_ptr(), _in_type(torch, values),
                                           q.data_ptr(), scale.data_ptr(), int(tiled), rows, cols,
                                           ops._stream())  # fmt: skip
        ops._check(code, "the mxfp8 encoder")
    params = {"block_size": MX_BLOCK, "scale_layout": scale_layout}
    sse, energy, worst = (0.0, 0.0, 0.0) if not rows else _measured(
        torch, ops, values, _decoded(torch, "mxfp8", params, {"weight": q, "scale": scale},
                                     (rows, cols), values.device))  # fmt: skip
    return Encoded("F8_E4M3", [rows, cols], q,
                   [Companion(".weight_scale", "F8_E8M0", shape, scale)], 0, sse, energy, worst)  # fmt: skip


def encode_w4a8(torch: Any, key: str, values: Tensor) -> Encoded:
    """w4a8.convrot with the fixed codebook (`derive/microscale.py:349-408`): payload codes
    [R, C/2], `.weight_s_rel` F8_E4M3 [R, C/16], `.weight_s_channel` F32 [R] and
    `.weight_codebook` F32 [16]."""
    ops, values, rows, cols = _prepare(torch, key, values, CONVROT_GROUP)
    device = values.device
    codebook = torch.tensor(W4A8_CODEBOOK, dtype=torch.float32, device=device)
    codes = torch.empty(rows, cols // 2, dtype=torch.uint8, device=device)
    group = torch.empty(rows, cols // W4A8_GROUP, dtype=torch.float8_e4m3fn, device=device)
    scale = torch.empty(rows, dtype=torch.float32, device=device)
    if rows:
        code = ops._lib.cozyq_encode_w4a8(ops.index, values.data_ptr(), _in_type(torch, values),
                                          codebook.data_ptr(), codes.data_ptr(), group.data_ptr(),
                                          scale.data_ptr(), rows, cols, ops._stream())  # fmt: skip
        ops._check(code, "the w4a8 encoder")
    sse, energy, worst = 0.0, 0.0, 0.0
    if rows:
        levels = torch.empty(rows, cols, dtype=torch.int8, device=device)
        code = ops._lib.cozyq_w4a8_unpack(ops.index, codes.data_ptr(), group.data_ptr(),
                                          codebook.data_ptr(), levels.data_ptr(), rows, cols,
                                          ops._stream())  # fmt: skip
        ops._check(code, "the w4a8 unpack")
        params = {"rotation": "kron_regular_h4", "rotation_size": CONVROT_GROUP}
        sse, energy, worst = _measured(torch, ops, values, _decoded(
            torch, "int8.convrot", params, {"weight": levels, "scale": scale}, (rows, cols), device))  # fmt: skip
    return Encoded("I8", [rows, cols // 2], codes, [
        Companion(".weight_s_rel", "F8_E4M3", [rows, cols // W4A8_GROUP], group),
        Companion(".weight_s_channel", "F32", [rows], scale),
        Companion(".weight_codebook", "F32", [16], codebook),
    ], 0, sse, energy, worst)  # fmt: skip


def encode_nvfp4(torch: Any, key: str, values: Tensor) -> Encoded:
    """nvfp4 (`derive/microscale.py:146-217`): payload U8 [R, C/2] (low nibble first),
    `.weight_scale` F8_E4M3 [R, C/16] row-major and `.weight_scale_2` F32 []."""
    ops, values, rows, cols = _prepare(torch, key, values, NVFP4_BLOCK)
    device = values.device
    if not cols:
        raise UnsupportedInput(f"{key!r}: NVFP4 requires nonempty weight columns")
    codes = torch.empty(rows, cols // 2, dtype=torch.uint8, device=device)
    scale = torch.empty(rows, cols // NVFP4_BLOCK, dtype=torch.uint8, device=device)
    second = torch.ones((), dtype=torch.float32, device=device)
    counters = torch.zeros(2, dtype=torch.int64, device=device)  # amax bits, saturated
    if rows:
        code = ops._lib.cozyq_encode_nvfp4(ops.index, values.data_ptr(), _in_type(torch, values),
                                           codes.data_ptr(), scale.data_ptr(), second.data_ptr(),
                                           counters.data_ptr(), counters.data_ptr() + 8, rows,
                                           cols, ops._stream())  # fmt: skip
        ops._check(code, "the nvfp4 encoder")
    sse, energy, worst, saturated = 0.0, 0.0, 0.0, 0
    if rows:
        params = {"block_size": NVFP4_BLOCK, "global_scale": "multiply",
                  "nibble_order": "low_first", "scale_layout": "row_major"}  # fmt: skip
        parts = {"weight": codes, "scale": scale.view(torch.float8_e4m3fn), "scale_2": second}
        sse, energy, worst = _measured(torch, ops, values, _decoded(
            torch, "nvfp4", params, parts, (rows, cols), device))  # fmt: skip
        saturated = int(counters[1].cpu())
    return Encoded("U8", [rows, cols // 2], codes, [
        Companion(".weight_scale", "F8_E4M3", [rows, cols // NVFP4_BLOCK], scale.view(torch.float8_e4m3fn)),
        Companion(".weight_scale_2", "F32", [], second),
    ], saturated, sse, energy, worst)  # fmt: skip


def _svdq_int4_dense(torch: Any, codes: Tensor, scales: Tensor, p: Tensor, down: Tensor,
                     up: Tensor) -> Tensor:
    """The float32 weight an svdq.int4g64 encoding stands for: codes · group scale, back out of
    the smoothed basis (· p), plus up·down — what `_measured` holds against the source."""
    rows, cols = int(codes.shape[0]), 2 * int(codes.shape[1])
    lo = (codes & 0xF).to(torch.int16)
    hi = (codes >> 4).to(torch.int16)
    q = torch.stack((lo, hi), dim=-1).reshape(rows, cols)
    q = torch.where(q >= 8, q - 16, q).float()
    v = (q.view(rows, -1, SVDQ_INT4_GROUP) * scales.float().unsqueeze(-1)).view(rows, cols)
    return v * p.float() + up.float() @ down.float()


def encode_svdq_int4(torch: Any, key: str, values: Tensor, p: Tensor, down: Tensor,
                     up: Tensor) -> Encoded:
    """svdq.int4g64 (this build's W4A4 variant; the reference's svdq writer is tensorfs's): the
    residual `values − up·down` moved into the smoothed basis (÷ p per input channel), int4 codes
    per 64-group with fp16 scales (`cozyq_encode_svdq_int4`). Payload U8 [R, C/2] (element 2k
    low), `.weight_scale` F16 [R, C/64], and the branch and smoothing it was encoded against:
    `.pre_quant_scale` F32 [C], `.lowrank_down` BF16 [r, C], `.lowrank_up` BF16 [R, r]."""
    ops, values, rows, cols = _prepare(torch, key, values, SVDQ_INT4_GROUP)
    device = values.device
    rank = int(down.shape[0])
    if tuple(down.shape) != (rank, cols) or tuple(up.shape) != (rows, rank):
        raise UnsupportedInput(f"{key!r}: the low-rank branch must be down [r, {cols}] and up [{rows}, r]")
    p = p.to(device=device, dtype=torch.float32).contiguous()
    down = down.to(device=device, dtype=torch.bfloat16).contiguous()
    up = up.to(device=device, dtype=torch.bfloat16).contiguous()
    if p.numel() != cols:
        raise UnsupportedInput(f"{key!r}: pre_quant_scale must hold {cols} values")
    codes = torch.empty(rows, cols // 2, dtype=torch.uint8, device=device)
    scales = torch.empty(rows, cols // SVDQ_INT4_GROUP, dtype=torch.float16, device=device)
    if rows:
        code = ops._lib.cozyq_encode_svdq_int4(ops.index, values.data_ptr(), _in_type(torch, values),
                                               p.data_ptr(), down.data_ptr(), up.data_ptr(), rank,
                                               codes.data_ptr(), scales.data_ptr(), rows, cols,
                                               ops._stream())  # fmt: skip
        ops._check(code, "the svdq int4 encoder")
    sse, energy, worst = (0.0, 0.0, 0.0) if not rows else _measured(
        torch, ops, values, _svdq_int4_dense(torch, codes, scales, p, down, up).contiguous())  # fmt: skip
    return Encoded("U8", [rows, cols // 2], codes, [
        Companion(".weight_scale", "F16", [rows, cols // SVDQ_INT4_GROUP], scales),
        Companion(".pre_quant_scale", "F32", [cols], p),
        Companion(".lowrank_down", "BF16", [rank, cols], down),
        Companion(".lowrank_up", "BF16", [rows, rank], up),
    ], 0, sse, energy, worst)  # fmt: skip

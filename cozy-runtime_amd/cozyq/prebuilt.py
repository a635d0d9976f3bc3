"""`Prebuilt`: the op library over the HIP kernels, one per card — cozyq's stand-in for
cozy-runtime's `internal/prebuilt.py:80-434` (`Prebuilt`), with the same method names, argument
meaning, validation and errors, plus the MXFP8 and int4-g64 SVDQuant ops the reference serves
through cuBLASLt and nvfp4 kernels respectively.

It allocates outputs with torch and launches on torch's current stream by raw pointer through
the C ABI (`_lib`). There is no fallback: a shape no kernel takes raises, and a missing library
raises `KernelsAbsent` when the op is opened (`library`). `torch` is imported lazily so the
module imports without it.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from functools import partial
from typing import Any

from cozyq import _lib, verify
from cozyq._admit import ALIGN, EXTENT, KIND, LAYOUT, ROWS, Operand, Placement, admit, every, off_card

Tensor = Any
Dtype = Any

#: The one tensor-core family this library carries (the reference's `FAMILIES`,
#: `_kernels/__init__.py`): CDNA4's MFMA on gfx950.
FAMILIES = ("mfma.cdna4",)
#: Rows the fused fp8 linear may take in one launch (`cozyq_fp8_linear`: up to 4 rows the GEMV,
#: 5 to 16 with K <= 4096 the row-tile kernel, which also takes 3-4 rows of a wide weight; it
#: answers NOT_SUPPORTED past that); more rows quantize once and run the GEMM.
FP8_SMALL_ROWS = 16
#: From 2 rows, and `GEMV_TWO_LAUNCH_AREA` rows x K up, the int8 linear quantizes once and runs
#: the GEMM (at 1..4 rows a GEMV on the quantized rows) instead of the one-launch GEMV (same
#: bits). Each one-launch workgroup rotates every row of x itself, so that work grows with rows x
#: K; measured on MI355X (graph replays over weights past the MALL, µs one launch / two):
#: K=3072 N=12288 M=1 9.2 / 12.5, M=2 11.8 / 13.3, M=3 18.0 / 14.0, M=4 22.4 / 15.3; K=4096
#: N=14336 M=2 16.0 / 17.9, M=4 27.3 / 20.7; K=12288 N=3072 M=2 18.0 / 14.9, M=4 28.4 / 16.7;
#: K=3072 N=3072 M=4 11.8 / 10.8; K=16384 N=4096 M=2 27.5 / 24.0; K=32768 N=4096 M=1 41.7 / 47.3.
GEMV_TWO_LAUNCH_ROWS = 2
GEMV_TWO_LAUNCH_AREA = 9216


def gemv_serves(rows: int, width: int) -> bool:
    """Whether the int8 linear of `rows` rows of `width` elements takes the one-launch GEMV
    (within its row range; it may still decline a width), rather than quantize + GEMM."""
    if rows >= GEMV_TWO_LAUNCH_ROWS and rows * width >= GEMV_TWO_LAUNCH_AREA:
        return False
    return True


#: The svdq low-rank ranks the kernels take.
RANKS = (16, 32, 64)
#: int4 SVDQuant K-group.
INT4_GROUP = 64
MX_BLOCK = 32


@dataclass(frozen=True, slots=True)
class _Format:
    name: str
    fp8: bool
    #: the activation width each row must be a multiple of
    multiple: int


#: `internal/prebuilt.py:68`: int8 rows rotate in 256-groups; fp8 rows are 16-byte multiples.
#: The prologue's gated activation codes (`internal/prebuilt.py` SITU / SWIGLU): x holds
#: [hidden | gate] (or, for SwiGLU without `up`, [up | gate]) halves.
SITU, SWIGLU = 3, 4

#: `w4a8_gemm`'s config that unpacks the codes once and multiplies on the int8 GEMM, and the
#: rows from which it is chosen (`internal/prebuilt.py:48-49`): past 256 rows the 256x256 int8
#: GEMM outruns the fused narrow-tile one, and the unpack is one pass over the weight. It is the
#: number of the 256x256 tile in the int8 GEMM's table, which the fused 4-bit GEMM lacks; the
#: fused GEMM's configs 1..4 are that table's narrow tiles.
UNPACK = 0
UNPACK_ROWS = 257
#: The GEMM tile configs (`cozyq_gemm`): 0 256x256, 1 128x128, 2 128x64, 3 64x64, 4 32x64,
#: 5 256x192.
GEMM_CONFIGS = 6
#: The configs with 256-row tiles, which `w4a8_gemm` runs by unpacking the codes first.
WIDE_TILES = (UNPACK, 5)

INT8, FP8 = _Format("int8", False, 256), _Format("fp8", True, 16)
MX = _Format("mxfp8", True, 128)
SVDQ = _Format("svdq-int4", False, INT4_GROUP)
#: svdq.nvfp4: K in whole 64-element GEMM steps (the reference's `kDepth`, svdq.h:15), and the
#: ranks its kernels take (`internal/svdq_linear.py:49`).
SVDQ_NVFP4 = _Format("svdq.nvfp4", False, 64)
NVFP4_RANKS = (32, 64, 128)


def _torch():
    import torch

    return torch


@dataclass(frozen=True)
class W4a8:
    """One `w4a8.convrot` weight as the GEMM reads it (`internal/prebuilt.py:437-446`): `codes`
    bytes [N, K/2] (even k in the low nibble), E4M3 `group_scale` [N, K/16], float32 row
    `scale` [N] and `codebook` [16] (None: the uniform grid `q - 8`)."""

    codes: Tensor
    group_scale: Tensor
    scale: Tensor
    codebook: Tensor | None


def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else int(t.data_ptr())


def _stride(t: Tensor | None) -> int:
    return 0 if t is None else int(t.stride(0))


def _aligned(t: Tensor) -> Tensor:
    """`t` contiguous at a 16-byte address: the epilogues read scales and biases 16 bytes at a
    time."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


@dataclass(slots=True)
class Prebuilt:
    """The ops on one card (`internal/prebuilt.py:80-434`)."""

    torch: Any
    index: int
    family: str = FAMILIES[0]
    _lib: Any = field(init=False)
    #: 16-bit dtype -> whether it is fp16 (the kernels' `half` flag).
    _halves: dict[Any, bool] = field(init=False, default_factory=dict)
    #: The fused linear's counters, one zeroed int32 buffer per stream (each call leaves its
    #: buffer zero; calls on one stream run in order, so they share it).
    _workspaces: dict[int, Tensor] = field(init=False, default_factory=dict)
    #: format -> its self-check on this card (`cozyq.verify`), set by `library`.
    verdicts: dict[str, Any] = field(init=False, default_factory=dict)

    def __post_init__(self) -> None:
        self._lib = _lib.load()
        self._halves = {self.torch.bfloat16: False, self.torch.float16: True}

    # ------------------------------------------------------------------ reference surface

    def int8_linear(
        self, x: Tensor, data: Tensor, scale: Tensor, bias: Tensor | None, out_dtype: Dtype
    ) -> Tensor:
        """`x @ W.T + bias` for an int8.convrot weight (`internal/prebuilt.py:99-117`): the
        one-launch GEMV where it takes the rows (`_gemv`), else quantize + GEMM. (Two launches
        also beat the fused one, `int8_linear_rot`, on MI355X: its quantize jobs run at one wave a
        SIMD beside the GEMM's full register file.)"""
        flat = self._rows(INT8, x)
        bias = self._weight(INT8, data, scale, bias, flat.shape[1], out_dtype)
        scale = _aligned(scale)
        shape = (*x.shape[:-1], data.shape[0])
        served = self._gemv(flat, data, scale, bias, out_dtype, shape)
        if served is not None:
            return served
        q, scales = self.int8_quantize(flat)
        return self.int8_gemm(q, scales, data, scale, bias, out_dtype).view(shape)

    def _gemv(self, flat: Tensor, data: Tensor, scale: Tensor, bias: Tensor | None,
              out_dtype: Dtype, shape: tuple[int, ...]) -> Tensor | None:  # fmt: skip
        """The whole int8 linear of up to `GEMV_ROWS` checked rows in one launch
        (`cozyq_gemv`), or None where it declines (more rows, rows too wide for it, or a shape
        where quantize + GEMM is faster, `gemv_serves`)."""
        rows, width = flat.shape
        if rows > self._lib.cozyq_gemv_rows() or not gemv_serves(rows, width):
            return None
        out = self.torch.empty(shape, dtype=out_dtype, device=flat.device)
        if rows == 0:
            return out
        code = self._lib.cozyq_gemv(
            self.index, flat.data_ptr(), self._half(flat.dtype), data.data_ptr(), scale.data_ptr(),
            _ptr(bias), out.data_ptr(), self._half(out_dtype), rows, data.shape[0], width,
            self._stream(),
        )  # fmt: skip
        if code == self._lib.cozyq_not_supported():
            return None
        self._check(code, "the GEMV")
        return out

    def _linear_fused(
        self, flat: Tensor, data: Tensor, scale: Tensor, bias: Tensor | None, out_dtype: Dtype,
        rotation: int, epilogue: int,
    ) -> tuple[Tensor, Tensor, Tensor] | None:
        """`cozyq_linear` on checked rows: (out, q, scales), or None where it declines (rows
        longer than 4096, or an output dtype other than x's) and quantize + GEMM serve."""
        torch = self.torch
        rows, width = flat.shape
        n = int(data.shape[0])
        out = torch.empty(rows, n, dtype=out_dtype, device=flat.device)
        q = torch.empty(rows, width, dtype=torch.int8, device=flat.device)
        scales = torch.empty(rows, dtype=torch.float32, device=flat.device)
        stream = self._stream()
        need = int(self._lib.cozyq_linear_workspace_bytes(rows)) // 4
        work = self._workspaces.get(stream)
        if work is None or work.numel() < need:
            work = self._workspaces[stream] = torch.zeros(max(need, 1024), dtype=torch.int32,
                                                          device=flat.device)  # fmt: skip
        code = self._lib.cozyq_linear(
            self.index, flat.data_ptr(), self._half(flat.dtype), rotation, q.data_ptr(),
            scales.data_ptr(), data.data_ptr(), scale.data_ptr(), _ptr(bias), out.data_ptr(), n,
            self._half(out_dtype), rows, n, width, epilogue, work.data_ptr(), stream,
        )  # fmt: skip
        if code == self._lib.cozyq_not_supported():
            return None
        self._check(code, "the fused linear")
        return out, q, scales

    def int8_linear_rot(
        self, x: Tensor, data: Tensor, scale: Tensor, bias: Tensor | None, out_dtype: Dtype,
        rotation: int, epilogue: int = 0, verify: bool = False,
    ) -> tuple[Tensor, Tensor, Tensor] | None:
        """The fused linear (`cozyq_linear`) for any rotation lane (256, 128, 0) and epilogue
        (0 none, 1 tanh-GELU): (out, q, scales) with q / scales the operand it quantized, or None
        where it declines. A tile whose wait for its rows gave up is written as NaN; `verify`
        synchronizes the stream after the call and raises RuntimeError if that happened."""
        multiple = 16 if rotation == 0 else rotation
        flat = self._rows(_Format("int8", False, multiple), x)
        bias = self._weight(_Format("int8", False, multiple), data, scale, bias, flat.shape[1], out_dtype)
        done = self._linear_fused(flat, data, _aligned(scale), bias, out_dtype, rotation, epilogue)
        if verify and done is not None:
            self.linear_status()
        return done

    def linear_status(self) -> None:
        """Raises RuntimeError if a fused linear on this stream's workspace gave up waiting for
        its rows since the last check (its tiles were written as NaN); synchronizes the stream
        and clears the record (`cozyq_linear_status`)."""
        stream = self._stream()
        work = self._workspaces.get(stream)
        if work is None:
            return
        self._check(self._lib.cozyq_linear_status(self.index, work.data_ptr(), stream),
                    "the fused linear (a tile's wait for its rows gave up)")  # fmt: skip

    def fp8_linear(
        self, x: Tensor, data: Tensor, scale: Tensor, bias: Tensor | None, out_dtype: Dtype
    ) -> Tensor:
        """`x @ W.T + bias` for an fp8.rowwise weight (`internal/prebuilt.py:119-124`). Up to
        `FP8_SMALL_ROWS` rows run as one fused launch (quantize + product) where the library takes
        the shape, the rest as two."""
        flat = self._rows(FP8, x)
        rows, width = flat.shape
        shape = (*x.shape[:-1], data.shape[0])
        if 0 < rows <= FP8_SMALL_ROWS:
            bias = self._weight(FP8, data, scale, bias, width, out_dtype)
            out = self.torch.empty(shape, dtype=out_dtype, device=x.device)
            code = self._lib.cozyq_fp8_linear(
                self.index, flat.data_ptr(), self._half(flat.dtype), data.data_ptr(),
                scale.data_ptr(), _ptr(bias), out.data_ptr(), self._half(out_dtype), rows,
                data.shape[0], width, self._stream(),
            )  # fmt: skip
            if code != self._lib.cozyq_not_supported():
                self._check(code, "the fp8 linear")
                return out
        q, scales = self.fp8_quantize(flat)
        return self.fp8_gemm(q, scales, data, scale, bias, out_dtype).view(shape)

    def int8_quantize(
        self, x: Tensor, scale: Tensor | None = None, shift: Tensor | None = None, norm: int = 0,
        eps: float = 0.0, activation: int = 0, up: Tensor | None = None,
    ) -> tuple[Tensor, Tensor]:
        return self._quantize(INT8, x, scale, shift, norm, eps, activation, up)

    def fp8_quantize(
        self, x: Tensor, scale: Tensor | None = None, shift: Tensor | None = None, norm: int = 0,
        eps: float = 0.0, activation: int = 0, up: Tensor | None = None,
    ) -> tuple[Tensor, Tensor]:
        return self._quantize(FP8, x, scale, shift, norm, eps, activation, up)

    def w4a8_linear(self, x: Tensor, w: W4a8, bias: Tensor | None, out_dtype: Dtype) -> Tensor:
        """`internal/prebuilt.py:176-178`: int8.convrot's operand, then `w4a8_gemm`."""
        q, scales = self.int8_quantize(x)
        return self.w4a8_gemm(q, scales, w, bias, out_dtype).view(*x.shape[:-1], w.codes.shape[0])

    def w4a8_gemm(
        self, q: Tensor, scales: Tensor, w: W4a8, bias: Tensor | None, out_dtype: Dtype,
        config: int = -1,
    ) -> Tensor:
        """`internal/prebuilt.py:180-222`: `q @ unpack(w).T`, both scales and the bias. From
        `UNPACK_ROWS` rows the codes unpack once to int8 and the int8 GEMM multiplies them
        (config `UNPACK`, or 5 for the 256x192 tile, else the int8 GEMM's shape rule); fewer rows
        take the fused GEMM. Every config is the same law, bit for bit."""
        torch = self.torch
        rows, width = self._operand("w4a8_gemm", torch.int8, q, scales)
        bias = self._w4a8_weight(w, bias, width, out_dtype)
        n = w.codes.shape[0]
        if config in WIDE_TILES or (config < 0 and rows >= UNPACK_ROWS):
            levels = torch.empty(n, width, dtype=torch.int8, device=q.device)
            code = self._lib.cozyq_w4a8_unpack(
                self.index, w.codes.data_ptr(), w.group_scale.data_ptr(), _ptr(w.codebook),
                levels.data_ptr(), n, width, self._stream(),
            )  # fmt: skip
            self._check(code, "the w4a8 unpack")
            return self.int8_gemm(q, scales, levels, w.scale, bias, out_dtype, config)
        out = torch.empty(rows, n, dtype=out_dtype, device=q.device)
        if rows == 0:
            return out
        code = self._lib.cozyq_w4a8_gemm(
            self.index, q.data_ptr(), scales.data_ptr(), w.codes.data_ptr(),
            w.group_scale.data_ptr(), _ptr(w.codebook), w.scale.data_ptr(), _ptr(bias),
            out.data_ptr(), self._half(out_dtype), rows, n, width, config, self._stream(),
        )  # fmt: skip
        if code == self._lib.cozyq_not_supported() and config >= 0:
            raise ValueError(f"w4a8_gemm: config {config} cannot take {rows}x{width}")
        self._check(code, "the w4a8 GEMM")
        return out

    def w4a8_unpack(self, w: W4a8) -> Tensor:
        """The int8 levels [N, K] of `w`'s codes (`cozyq_w4a8_unpack`)."""
        n, width = w.codes.shape[0], 2 * w.codes.shape[1]
        self._w4a8_weight(w, None, width, self.torch.bfloat16)
        levels = self.torch.empty(n, width, dtype=self.torch.int8, device=w.codes.device)
        code = self._lib.cozyq_w4a8_unpack(
            self.index, w.codes.data_ptr(), w.group_scale.data_ptr(), _ptr(w.codebook),
            levels.data_ptr(), n, width, self._stream(),
        )  # fmt: skip
        self._check(code, "the w4a8 unpack")
        return levels

    def _w4a8_weight(self, w: W4a8, bias: Tensor | None, width: int, out_dtype: Dtype) -> Tensor | None:
        """Contract V5 (`internal/prebuilt.py:224-251`): the w4a8 weight's tensors, and `bias`
        in the output dtype."""
        torch = self.torch
        n = int(w.codes.shape[0])
        shapes = (f"w4a8: codes, group scales and scale must be [{n}, {width // 2}], "
                  f"[{n}, {width // 16}] and [{n}], contiguous")  # fmt: skip
        kinds = "w4a8: codes are bytes and group scales E4M3"
        packing = "w4a8: scale is float32, N a multiple of 8, codes 16-byte aligned"
        admit(
            (w.codes, Operand(itemsize=1, extents=(n, width // 2), dense=True, align=16, rows=8),
             {**every(shapes, EXTENT, LAYOUT), KIND: kinds, **every(packing, ALIGN, ROWS)}),
            (w.group_scale, Operand(kinds=(torch.float8_e4m3fn,), extents=(n, width // 16), dense=True, align=4),
             {**every(shapes, EXTENT, LAYOUT), KIND: kinds, ALIGN: "w4a8: group scales must be 4-byte aligned"}),
            (w.scale, Operand(kinds=(torch.float32,), extents=(n,), dense=True),
             {**every(shapes, EXTENT, LAYOUT), KIND: packing}),
        )  # fmt: skip
        if w.codebook is not None:
            admit((w.codebook, Operand(kinds=(torch.float32,), count=16),
                   every("w4a8: the codebook is 16 float32 levels", KIND, EXTENT)))  # fmt: skip
        if off_card(self.index, w.codes, w.group_scale, w.scale, w.codebook, bias):
            raise ValueError(f"w4a8: the weight's tensors must be on cuda:{self.index}")
        self._half(out_dtype)
        if bias is not None and bias.numel() != n:
            raise ValueError(f"w4a8: bias must have {n} values")
        return None if bias is None else bias.to(out_dtype).contiguous()

    def int8_gemm(
        self, q: Tensor, scales: Tensor, data: Tensor, scale: Tensor, bias: Tensor | None,
        out_dtype: Dtype, config: int = -1, out: Tensor | None = None,
    ) -> Tensor:
        return self._gemm(INT8, q, scales, data, scale, bias, out_dtype, config, out)

    def fp8_gemm(
        self, q: Tensor, scales: Tensor, data: Tensor, scale: Tensor, bias: Tensor | None,
        out_dtype: Dtype, config: int = -1, out: Tensor | None = None,
    ) -> Tensor:
        return self._gemm(FP8, q, scales, data, scale, bias, out_dtype, config, out)

    # ---------------------------------------------------------------- build extensions

    def int8_quantize_rot(self, x: Tensor, rotation: int) -> tuple[Tensor, Tensor]:
        """Per-token int8 with rotation 256 (the reference's), 128 (H2⊗H4⊗H4⊗H4, 1/√128 folded
        into the scale) or 0 (none): `cozyq_quantize_rot`."""
        torch = self.torch
        multiple = 16 if rotation == 0 else rotation
        flat = self._rows(_Format("int8", False, multiple), x)
        rows, width = flat.shape
        q = torch.empty(rows, width, dtype=torch.int8, device=x.device)
        scales = torch.empty(rows, dtype=torch.float32, device=x.device)
        code = self._lib.cozyq_quantize_rot(
            self.index, flat.data_ptr(), self._half(flat.dtype), q.data_ptr(), scales.data_ptr(),
            rows, width, rotation, self._stream(),
        )  # fmt: skip
        self._check(code, "the quantization")
        return q, scales

    def int8_gemm_ex(
        self, q: Tensor, scales: Tensor, data: Tensor, scale: Tensor, bias: Tensor | None,
        out_dtype: Dtype, epilogue: int = 0, out: Tensor | None = None,
    ) -> Tensor:
        """`int8_gemm` for any rotation lane (K % 16), with an epilogue activation
        (0 none, 1 tanh-GELU)."""
        return self._gemm(_Format("int8", False, 16), q, scales, data, scale, bias, out_dtype,
                          -1, out, epilogue)  # fmt: skip

    def int8_acc(self, q: Tensor, data: Tensor) -> Tensor:
        """The raw int32 `q @ dataᵀ` of the int8 MFMA mainloop (test entry)."""
        torch = self.torch
        rows, width = q.shape
        acc = torch.empty(rows, data.shape[0], dtype=torch.int32, device=q.device)
        code = self._lib.cozyq_gemm_i32(
            self.index, q.data_ptr(), data.data_ptr(), acc.data_ptr(), rows, data.shape[0], width,
            self._stream(),
        )  # fmt: skip
        self._check(code, "the int32 GEMM")
        return acc

    def mx_quantize(self, x: Tensor) -> tuple[Tensor, Tensor]:
        """`leaves.quantize_activation_mx`'s law (`internal/encoding/leaves.py:1411-1424`):
        e4m3 `[M, K]` and row-major E8M0 bytes `[M, K/32]`."""
        torch = self.torch
        flat = self._rows(_Format("mxfp8", True, MX_BLOCK), x)
        rows, width = flat.shape
        q = torch.empty(rows, width, dtype=torch.float8_e4m3fn, device=x.device)
        scales = torch.empty(rows, width // MX_BLOCK, dtype=torch.uint8, device=x.device)
        code = self._lib.cozyq_mx_quantize(
            self.index, flat.data_ptr(), self._half(flat.dtype), q.data_ptr(), scales.data_ptr(),
            rows, width, self._stream(),
        )  # fmt: skip
        self._check(code, "the MX quantization")
        return q, scales

    def mx_gemm(
        self, q: Tensor, qscales: Tensor, data: Tensor, wscales: Tensor, bias: Tensor | None,
        out_dtype: Dtype, out: Tensor | None = None,
    ) -> Tensor:
        """`_scaled_mm` with 1x32 E8M0 block scales (`internal/encoding/leaves.py:1509-1519`) on
        the scaled MFMA; scale grids row-major `[rows, K/32]`."""
        torch = self.torch
        if q.dtype != torch.float8_e4m3fn or q.dim() != 2 or not q.is_contiguous():
            raise ValueError("mx_gemm: q must be a contiguous e4m3 [M, K]")
        rows, width = q.shape
        if width % MX.multiple:
            raise ValueError(f"mx_gemm: K must be a multiple of {MX.multiple}, not {width}")
        n = data.shape[0]
        grid = (width // MX_BLOCK,)
        if qscales.dtype not in (torch.uint8, torch.float8_e8m0fnu) or tuple(qscales.shape) != (rows, *grid):
            raise ValueError(f"mx_gemm: q scales must be E8M0 bytes [{rows}, {grid[0]}]")
        if data.dtype != torch.float8_e4m3fn or tuple(data.shape) != (n, width) or not data.is_contiguous():
            raise ValueError(f"mx_gemm: data must be a contiguous e4m3 [N, {width}]")
        if wscales.dtype not in (torch.uint8, torch.float8_e8m0fnu) or tuple(wscales.shape) != (n, *grid):
            raise ValueError(f"mx_gemm: weight scales must be E8M0 bytes [{n}, {grid[0]}]")
        if n % 8:
            raise ValueError("mx_gemm: N must be a multiple of 8")
        self._half(out_dtype)
        bias = None if bias is None else bias.to(out_dtype).contiguous()
        direct = out is not None and Placement(rows, n, out_dtype, q.device).takes(out)
        result = out if direct else torch.empty(rows, n, dtype=out_dtype, device=q.device)
        if rows == 0:
            return _landed(result, out)
        code = self._lib.cozyq_mx_gemm(
            self.index, q.data_ptr(), qscales.contiguous().data_ptr(), data.data_ptr(),
            wscales.contiguous().data_ptr(), _ptr(bias), result.data_ptr(), result.stride(0),
            self._half(out_dtype), rows, n, width, self._stream(),
        )  # fmt: skip
        self._check(code, "the MX GEMM")
        return _landed(result, out)

    def mx_linear(
        self, x: Tensor, data: Tensor, wscales: Tensor, bias: Tensor | None, out_dtype: Dtype
    ) -> Tensor:
        q, qs = self.mx_quantize(x)
        out = self.mx_gemm(q, qs, data, wscales, bias, out_dtype)
        return out.view(*x.shape[:-1], data.shape[0])

    def svdq_int4_quantize(
        self, x: Tensor, p: Tensor, down: Tensor
    ) -> tuple[Tensor, Tensor, Tensor]:
        """The int4-g64 activation side (`cozyq_svdq_int4_quantize`): packed codes `[M, K/2]`,
        fp16 group scales `[M, K/64]` and the low-rank input `bf16(x·downᵀ)` `[M, R]`."""
        torch = self.torch
        flat = self._rows(SVDQ, x)
        rows, width = flat.shape
        r = int(down.shape[0])
        if r not in RANKS or tuple(down.shape) != (r, width) or down.dtype != torch.bfloat16:
            raise ValueError(f"svdq: down must be bf16 [R, {width}], R in {RANKS}")
        if p.dtype != torch.float32 or p.numel() != width:
            raise ValueError(f"svdq: p must be float32 with {width} values")
        act = torch.empty(rows, width // 2, dtype=torch.uint8, device=x.device)
        ascales = torch.empty(rows, width // INT4_GROUP, dtype=torch.float16, device=x.device)
        la = torch.empty(rows, r, dtype=torch.bfloat16, device=x.device)
        if rows == 0:
            return act, ascales, la
        code = self._lib.cozyq_svdq_int4_quantize(
            self.index, flat.data_ptr(), self._half(flat.dtype), _aligned(p).data_ptr(),
            _aligned(down).data_ptr(), act.data_ptr(), ascales.data_ptr(), la.data_ptr(), rows,
            width, r, self._stream(),
        )  # fmt: skip
        self._check(code, "the svdq quantization")
        return act, ascales, la

    def svdq_int4_gemm(
        self, act: Tensor, ascales: Tensor, la: Tensor, w: Tensor, wscales: Tensor, up: Tensor,
        bias: Tensor | None, out_dtype: Dtype,
    ) -> Tensor:
        """The int4-g64 GEMM (`cozyq_svdq_int4_gemm`) with the low-rank term and the bias."""
        torch = self.torch
        rows, width = int(act.shape[0]), 2 * int(act.shape[1])
        n, r = int(w.shape[0]), int(up.shape[1])
        if tuple(w.shape) != (n, width // 2) or tuple(wscales.shape) != (n, width // INT4_GROUP):
            raise ValueError(f"svdq: weight codes [N, {width // 2}] and scales [N, {width // INT4_GROUP}]")
        if tuple(up.shape) != (n, r) or up.dtype != torch.bfloat16 or tuple(la.shape) != (rows, r):
            raise ValueError("svdq: up must be bf16 [N, R] and la [M, R]")
        if n % 8:
            raise ValueError("svdq: N must be a multiple of 8")
        if act.dtype != torch.uint8 or w.dtype != torch.uint8 or la.dtype != torch.bfloat16:
            raise ValueError("svdq: codes must be uint8 (two int4 a byte) and la bf16")
        if ascales.dtype != torch.float16 or wscales.dtype != torch.float16:
            raise ValueError("svdq: group scales must be float16")
        if tuple(ascales.shape) != (rows, width // INT4_GROUP):
            raise ValueError(f"svdq: activation scales must be [{rows}, {width // INT4_GROUP}]")
        self._half(out_dtype)
        bias = None if bias is None else _aligned(bias.to(out_dtype))
        out = torch.empty(rows, n, dtype=out_dtype, device=act.device)
        if rows == 0:
            return out
        act, ascales, w, wscales, la, up = (
            _aligned(t) for t in (act, ascales, w, wscales, la, up))
        code = self._lib.cozyq_svdq_int4_gemm(
            self.index, act.data_ptr(), ascales.data_ptr(), w.data_ptr(), wscales.data_ptr(),
            la.data_ptr(), up.data_ptr(), _ptr(bias), out.data_ptr(),
            self._half(out_dtype), rows, n, width, r, self._stream(),
        )  # fmt: skip
        self._check(code, "the svdq GEMM")
        return out

    def svdq_int4_linear(
        self, x: Tensor, p: Tensor, down: Tensor, w: Tensor, wscales: Tensor, up: Tensor,
        bias: Tensor | None, out_dtype: Dtype,
    ) -> Tensor:
        act, ascales, la = self.svdq_int4_quantize(x, p, down)
        out = self.svdq_int4_gemm(act, ascales, la, w, wscales, up, bias, out_dtype)
        return out.view(*x.shape[:-1], w.shape[0])

    # ----------------------------------------------------------- svdq.nvfp4 W4A4

    def svdq_input_scale(self, x: Tensor, p: Tensor) -> Tensor:
        """g_x on the card (`cozyq_svdq_input_scale`; the reference's `activation_scale`,
        `internal/svdq_linear.py:582-590`, without a stored `input_scale`): float32 [1]."""
        torch = self.torch
        flat = self._rows(SVDQ_NVFP4, x)
        rows, width = flat.shape
        if p.dtype != torch.float32 or p.numel() != width:
            raise ValueError(f"svdq: p must be float32 with {width} values")
        g = torch.empty(1, dtype=torch.float32, device=x.device)
        code = self._lib.cozyq_svdq_input_scale(
            self.index, flat.data_ptr(), self._half(flat.dtype), _aligned(p).data_ptr(), rows,
            width, g.data_ptr(), self._stream())  # fmt: skip
        self._check(code, "the svdq input scale")
        return g

    def svdq_quantize(
        self, x: Tensor, p: Tensor, g: Tensor, down: Tensor
    ) -> tuple[Tensor, Tensor, Tensor]:
        """`svdq_quantize` (`internal/svdq_linear.py:510-534`, `kernels/csrc/gemm.cpp:169-178`):
        x's nvfp4 operand at second level g — codes `[Rows(M), K/2]` (u8, element 2k low) and
        E4M3 scales `[Rows(M), K/16]` — and the low-rank input `bf16(x·downᵀ)` `[Rows(M), R]`,
        rows past M zero (Rows(M) = M rounded up to 256)."""
        torch = self.torch
        flat = self._rows(SVDQ_NVFP4, x)
        rows, width = flat.shape
        r = int(down.shape[0])
        if r not in NVFP4_RANKS or tuple(down.shape) != (r, width) or down.dtype != torch.bfloat16:
            raise ValueError(f"svdq: down must be bf16 [R, {width}], R in {NVFP4_RANKS}")
        if p.dtype != torch.float32 or p.numel() != width:
            raise ValueError(f"svdq: p must be float32 with {width} values")
        if g.dtype != torch.float32 or g.numel() != 1 or g.device != x.device:
            raise ValueError("svdq: g must be one float32 on x's device")
        padded = self._lib.cozyq_svdq_rows(rows)
        act = torch.empty(padded, width // 2, dtype=torch.uint8, device=x.device)
        ascales = torch.empty(padded, width // 16, dtype=torch.float8_e4m3fn, device=x.device)
        la = torch.empty(padded, r, dtype=torch.bfloat16, device=x.device)
        code = self._lib.cozyq_svdq_quantize(
            self.index, flat.data_ptr(), self._half(flat.dtype), _aligned(p).data_ptr(),
            g.data_ptr(), _aligned(down).data_ptr(), act.data_ptr(), ascales.data_ptr(),
            la.data_ptr(), rows, width, r, self._stream(),
        )  # fmt: skip
        self._check(code, "the svdq quantization")
        return act, ascales, la

    def svdq_gemm(
        self, act: Tensor, ascales: Tensor, la: Tensor, rows: int, gx: Tensor, weight: Tensor,
        scale: Tensor, scale_2: Tensor, up: Tensor, c: Tensor | None, bias: Tensor | None,
        out_dtype: Dtype,
    ) -> Tensor:
        """`svdq_gemm` (`internal/svdq_linear.py:537-567`, `kernels/csrc/gemm.cpp:180-190`):
        `[rows, N]` = `(A·Wᵀ)·gx·gw·c + la·upᵀ + bias`, rounded once. `weight` u8 `[N, K/2]`
        and `scale` E4M3 `[N, K/16]` as stored; `scale_2` (gw) and `gx` float32 [1]; `up` bf16
        `[N, R]`; `c` float32 `[N]` or None."""
        torch = self.torch
        width = 2 * int(act.shape[1])
        n, r = int(weight.shape[0]), int(up.shape[1])
        if tuple(weight.shape) != (n, width // 2) or tuple(scale.shape) != (n, width // 16):
            raise ValueError(f"svdq: weight [N, {width // 2}] and scale [N, {width // 16}]")
        if weight.dtype != torch.uint8 or scale.dtype != torch.float8_e4m3fn:
            raise ValueError("svdq: the weight is uint8 codes with float8_e4m3fn scales")
        if r not in NVFP4_RANKS or tuple(up.shape) != (n, r) or up.dtype != torch.bfloat16:
            raise ValueError(f"svdq: up must be bf16 [N, R], R in {NVFP4_RANKS}")
        if tuple(la.shape) != (int(act.shape[0]), r) or la.dtype != torch.bfloat16:
            raise ValueError("svdq: la must be bf16 [Rows(M), R]")
        if n % 8:
            raise ValueError("svdq: N must be a multiple of 8")
        if c is not None and (c.dtype != torch.float32 or c.numel() != n):
            raise ValueError(f"svdq: channel_scale must be float32 with {n} values")
        half = self._half(out_dtype)
        out = torch.empty(rows, n, dtype=out_dtype, device=act.device)
        if rows == 0:
            return out
        bias = None if bias is None else _aligned(bias.to(out_dtype).reshape(-1))
        tensors = (act, ascales, weight, scale, la, up)
        act, ascales, weight, scale, la, up = (_aligned(t) for t in tensors)
        gw = scale_2.to(torch.float32).reshape(1)
        code = self._lib.cozyq_svdq_gemm(
            self.index, act.data_ptr(), ascales.data_ptr(), weight.data_ptr(), scale.data_ptr(),
            gx.data_ptr(), gw.data_ptr(), _ptr(None if c is None else _aligned(c)), la.data_ptr(),
            up.data_ptr(), _ptr(bias), out.data_ptr(), half, rows, n, width, r, self._stream(),
        )  # fmt: skip
        self._check(code, "the svdq GEMM")
        return out

    def svdq_linear(self, x: Tensor, roles: dict, bias: Tensor | None, out_dtype: Dtype) -> Tensor:
        """The svdq.nvfp4 linear (`internal/svdq_linear.py:662-697` on the prebuilt kernels):
        g_x (the stored `input_scale`, else `svdq_input_scale`), `svdq_quantize`, `svdq_gemm`.
        `roles` as the reference's leaf holds them: `weight`, `scale`, `scale_2`,
        `pre_quant_scale`, `lowrank_down`, `lowrank_up`, optional `channel_scale` and
        `input_scale`."""
        torch = self.torch
        p = roles["pre_quant_scale"]
        flat = self._rows(SVDQ_NVFP4, x)
        stored = roles.get("input_scale")
        g = self.svdq_input_scale(flat, p) if stored is None else stored.to(torch.float32).reshape(1)
        act, ascales, la = self.svdq_quantize(flat, p, g, roles["lowrank_down"])
        out = self.svdq_gemm(act, ascales, la, int(flat.shape[0]), g, roles["weight"],
                             roles["scale"], roles["scale_2"], roles["lowrank_up"],
                             roles.get("channel_scale"), bias, out_dtype)  # fmt: skip
        return out.view(*x.shape[:-1], -1)

    # ------------------------------------------------------------------- nvfp4 W4A16

    def nvfp4_gemv(self, x: Tensor, weight: Tensor, blocked_scale: Tensor, scale_2: Tensor,
                   out_dtype: Dtype) -> Tensor:
        """`cozyq_nvfp4_gemv` (the `_gemv` path of `internal/nvfp4_linear.py:126-201`, and the
        decode + GEMM path of `:376-385` up to 64 rows): up to 64 bf16/fp16 rows against packed
        E2M1 codes [N, K/2] (low nibble first), E4M3 scales in cuBLAS's 128x4 tiles and a float32
        second level; out [M, N] in `out_dtype` (bf16/fp16)."""
        torch = self.torch
        flat = x.reshape(-1, x.shape[-1])
        rows, cols = int(flat.shape[0]), int(flat.shape[1])
        n = int(weight.shape[0])
        if rows > 64 or cols % 32 or 2 * int(weight.shape[1]) != cols:
            raise ValueError(f"nvfp4 GEMV: up to 64 rows and K % 32 == 0 matching the weight's "
                             f"{2 * int(weight.shape[1])} columns; got [{rows}, {cols}]")  # fmt: skip
        flat = flat if flat.is_contiguous() and flat.data_ptr() % 16 == 0 else flat.contiguous().clone()
        out = torch.empty(rows, n, dtype=out_dtype, device=x.device)
        code = self._lib.cozyq_nvfp4_gemv(
            self.index, flat.data_ptr(), self._half(flat.dtype), weight.data_ptr(),
            blocked_scale.data_ptr(), scale_2.data_ptr(), out.data_ptr(), self._half(out_dtype),
            rows, n, cols, self._stream(),
        )  # fmt: skip
        self._check(code, "the nvfp4 GEMV")
        return out

    def nvfp4_gemm(self, x: Tensor, weight: Tensor, blocked_scale: Tensor, scale_2: Tensor,
                   bias: Tensor | None, out_dtype: Dtype) -> Tensor:
        """`cozyq_nvfp4_gemm` (the decode-then-GEMM path of `internal/nvfp4_linear.py:376-385` as
        one kernel): bf16/fp16 rows against `nvfp4_gemv`'s operands, W decoded exactly into x's
        dtype on the matrix core, × scale_2 (+ bias) in the epilogue; K % 64 == 0, N % 8 == 0."""
        torch = self.torch
        flat = x.reshape(-1, x.shape[-1])
        rows, cols = int(flat.shape[0]), int(flat.shape[1])
        n = int(weight.shape[0])
        if cols % 64 or n % 8 or 2 * int(weight.shape[1]) != cols:
            raise ValueError(f"nvfp4 GEMM: K % 64 == 0 and N % 8 == 0 matching the weight's "
                             f"[{n}, {2 * int(weight.shape[1])}]; got [{rows}, {cols}]")  # fmt: skip
        if int(blocked_scale.numel()) < -(-n // 128) * 128 * (cols // 16):
            raise ValueError("nvfp4 GEMM: block scales must cover whole 128-row tiles")
        flat = flat if flat.is_contiguous() and flat.data_ptr() % 16 == 0 else flat.contiguous().clone()
        weight, blocked_scale = _aligned(weight), _aligned(blocked_scale)
        if bias is not None:
            bias = _aligned(bias.to(out_dtype))
        out = torch.empty(rows, n, dtype=out_dtype, device=x.device)
        code = self._lib.cozyq_nvfp4_gemm(
            self.index, flat.data_ptr(), self._half(flat.dtype), weight.data_ptr(),
            blocked_scale.data_ptr(), scale_2.data_ptr(), None if bias is None else bias.data_ptr(),
            out.data_ptr(), self._half(out_dtype), rows, n, cols, self._stream(),
        )  # fmt: skip
        self._check(code, "the nvfp4 GEMM")
        return out

    # -------------------------------------------------------------- stored-format decode

    def decode_table(
        self, code: int, weight: Tensor, scale: Tensor, scale_type: int, out: Tensor, rows: int,
        cols: int, *, grid: int, block: int = 1, tiled: bool = False,
        scale_2: Tensor | None = None, per_matrix: bool = False, divide: bool = False,
        post: Tensor | None = None, post_type: int = 0, high_first: bool = False,
        matrices: int = 1,
    ) -> None:
        """`cozyq_decode` into `out`: `matrices` stacked `[rows, cols]` matrices, the element
        law of `internal/encoding/formats.py:438-868` and `internal/decode_cores.py:196-230`.
        Parts are contiguous on `out`'s device; `post` is one factor or one per column."""
        post_mode = 0 if post is None else (2 if post.numel() == cols and cols != 1 else 1)
        second = 0 if scale_2 is None else (2 if divide else 1)
        code = self._lib.cozyq_decode(
            self.index, code, weight.data_ptr(), scale.data_ptr(), scale_type, grid, block,
            int(tiled), _ptr(scale_2), int(per_matrix), second, _ptr(post), post_type, post_mode,
            int(high_first), out.data_ptr(), _out_type(self.torch, out.dtype), rows, cols,
            matrices, self._stream(),
        )  # fmt: skip
        self._check(code, "the decode")

    def decode_convrot(
        self, weight: Tensor, scale: Tensor, scale_type: int, size: int, out: Tensor, rows: int,
        cols: int,
    ) -> None:
        """`cozyq_decode_convrot` into `out` (`internal/encoding/formats.py:733-752`)."""
        code = self._lib.cozyq_decode_convrot(
            self.index, weight.data_ptr(), scale.data_ptr(), scale_type, size, out.data_ptr(),
            _out_type(self.torch, out.dtype), rows, cols, self._stream(),
        )  # fmt: skip
        self._check(code, "the int8.convrot decode")

    def decode_svdq(
        self, weight: Tensor, scale: Tensor, tiled: bool, high_first: bool, scale_2: Tensor,
        divide: bool, channel: Tensor | None, channel_type: int, smooth: Tensor,
        smooth_type: int, down: Tensor, down_type: int, up: Tensor, up_type: int, out: Tensor,
        rows: int, cols: int,
    ) -> None:
        """`cozyq_decode_svdq` into `out` (`internal/decode_schemes.py:464-489`)."""
        code = self._lib.cozyq_decode_svdq(
            self.index, weight.data_ptr(), scale.data_ptr(), int(tiled), int(high_first),
            scale_2.data_ptr(), int(divide), _ptr(channel), channel_type, smooth.data_ptr(),
            smooth_type, down.data_ptr(), down_type, up.data_ptr(), up_type, int(down.shape[0]),
            out.data_ptr(), _out_type(self.torch, out.dtype), rows, cols, self._stream(),
        )  # fmt: skip
        self._check(code, "the svdq.nvfp4 decode")

    # ---------------------------------------------------------------------- internals

    def _quantize(
        self, f: _Format, x: Tensor, scale: Tensor | None, shift: Tensor | None, norm: int,
        eps: float, activation: int, up: Tensor | None,
    ) -> tuple[Tensor, Tensor]:
        """`internal/prebuilt.py:252-291`: per-row quantization with the producer prologue
        `activation(norm(x)·(1 + scale) + shift)` folded in. A gated row (SiTU, or SwiGLU
        without `up`) quantizes to half its width."""
        torch = self.torch
        # Contract V6: which prologues a call may combine.
        gated = activation == SITU or (activation == SWIGLU and up is None)
        width = x.shape[-1] // 2 if gated else x.shape[-1]
        flat = self._rows(f, x, width)
        rows = flat.shape[0]
        plain = not norm and scale is None and shift is None
        refusals = (
            (gated and (x.shape[-1] % 2 or not plain),
             f"{f.name}_quantize: a gated activation takes [hidden | gate] rows alone"),
            (up is not None and (activation != SWIGLU or up.shape != x.shape or up.dtype != x.dtype or not plain),
             f"{f.name}_quantize: SwiGLU takes gate and up rows of one shape alone"),
        )  # fmt: skip
        for refused, text in refusals:
            if refused:
                raise ValueError(text)
        other = None if up is None else self._rows(f, up)
        q = torch.empty(rows, width, dtype=torch.float8_e4m3fn if f.fp8 else torch.int8,
                        device=x.device)  # fmt: skip
        scales = torch.empty(rows, dtype=torch.float32, device=x.device)
        tables = [self._table(t, flat) for t in (scale, shift)]
        entries = next((t.shape[0] for t in tables if t is not None), rows) or 1
        if any(t is not None and t.shape[0] != entries for t in tables) or rows % entries:
            raise ValueError(f"{f.name}_quantize: modulation rows do not divide {rows} rows")
        code = self._lib.cozyq_quantize(
            self.index, f.fp8, flat.data_ptr(), self._half(flat.dtype), q.data_ptr(),
            scales.data_ptr(), rows, width, _ptr(tables[0]), _ptr(tables[1]),
            _stride(tables[0]), _stride(tables[1]), max(rows // entries, 1), norm, eps,
            activation, _ptr(other), self._stream(),
        )  # fmt: skip
        self._check(code, "the quantization")
        return q, scales

    def _table(self, table: Tensor | None, flat: Tensor) -> Tensor | None:
        """`internal/prebuilt.py:408-417`: a modulation table as `[E, K]` rows read 16 bytes at
        a time."""
        if table is None:
            return None
        if table.device != flat.device or table.dtype != flat.dtype:
            raise ValueError("a modulation table must match the activation's device and dtype")
        found = table.reshape(-1, flat.shape[1])
        if found.stride(1) != 1 or found.stride(0) % 8 or found.data_ptr() % 16:
            found = found.contiguous()
        return found if found.data_ptr() % 16 == 0 else found.clone()

    def _gemm(
        self, f: _Format, q: Tensor, scales: Tensor, data: Tensor, scale: Tensor,
        bias: Tensor | None, out_dtype: Dtype, config: int, out: Tensor | None = None,
        epilogue: int = 0,
    ) -> Tensor:
        """`internal/prebuilt.py:293-358`: `[M, N]` into `out` where given, written in place when
        its rows sit 16-byte multiples apart, else copied into it."""
        torch = self.torch
        rows, width = self._operand(f"{f.name}_gemm", torch.float8_e4m3fn if f.fp8 else torch.int8, q, scales)
        if width % f.multiple:
            raise ValueError(f"{f.name}_gemm: K must be a multiple of {f.multiple}, not {width}")
        bias = self._weight(f, data, scale, bias, width, out_dtype)
        scale = _aligned(scale)
        n = data.shape[0]
        direct = out is not None and Placement(rows, n, out_dtype, q.device).takes(out)
        result = out if direct and out is not None else torch.empty(
            rows, n, dtype=out_dtype, device=q.device)
        if rows == 0:
            return _landed(result, out)
        if epilogue == 0 and f in (INT8, FP8):
            code = self._lib.cozyq_gemm(
                self.index, FAMILIES.index(self.family), f.fp8, q.data_ptr(), scales.data_ptr(),
                data.data_ptr(), scale.data_ptr(), _ptr(bias), result.data_ptr(),
                result.stride(0), self._half(out_dtype), rows, n, width, config, None, None,
                self._stream(),
            )  # fmt: skip
        else:
            code = self._lib.cozyq_gemm_ex(
                self.index, f.fp8, q.data_ptr(), scales.data_ptr(), data.data_ptr(),
                scale.data_ptr(), _ptr(bias), result.data_ptr(), result.stride(0),
                self._half(out_dtype), rows, n, width, epilogue, self._stream(),
            )  # fmt: skip
        if code == self._lib.cozyq_not_supported() and config >= 0:
            raise ValueError(f"{f.name}_gemm: config {config} cannot take {rows}x{width}")
        self._check(code, "the GEMM")
        return _landed(result, out)

    def _operand(self, op: str, code: Dtype, q: Tensor, scales: Tensor) -> tuple[int, int]:
        """Contract V3: a quantized operand, codes `q` [M, K] and float32 row scales; (M, K)."""
        admit((q, Operand(kinds=(code,), extents=(None, None), dense=True, align=16),
               every(f"{op}: q must be a contiguous, aligned {code} [M, K]")))  # fmt: skip
        rows, width = (int(d) for d in q.shape)
        admit((scales, Operand(kinds=(self.torch.float32,), count=rows, dense=True),
               every(f"{op}: scales must be contiguous float32 with {rows} values")))  # fmt: skip
        return rows, width

    def _rows(self, f: _Format, x: Tensor, width: int | None = None) -> Tensor:
        """Contract V1 (`internal/prebuilt.py:360-370`): x on this card, each row quantizing to
        `width` elements (x's last extent unless given) that the kernels take; the rows as one
        contiguous matrix at a 16-byte address."""
        width = int(x.shape[-1] if width is None else width)
        limit = int(self._lib.cozyq_max_k())
        if off_card(self.index, x):
            raise ValueError(f"{f.name}: x must be on cuda:{self.index}")
        if width > limit or width % f.multiple:
            raise ValueError(f"{f.name}: K must be a multiple of {f.multiple} up to {limit}, not {width}")
        return _aligned(x.reshape(-1, x.shape[-1]))

    def _weight(
        self, f: _Format, data: Tensor, scale: Tensor, bias: Tensor | None, width: int,
        out_dtype: Dtype,
    ) -> Tensor | None:
        """Contract V2 (`internal/prebuilt.py:372-406`): an 8-bit weight (codes [N, width] and
        float32 row scales) on this card, a 16-bit output dtype, and `bias` in it."""
        torch = self.torch
        code = torch.float8_e4m3fn if f.fp8 else torch.int8
        admit((data, Operand(kinds=(code,), extents=(None, width), dense=True, align=16, rows=8),
               {**every(f"{f.name}: data must be {code} [N, {width}]", KIND, EXTENT),
                **every(f"{f.name}: data must be contiguous, aligned, N a multiple of 8", LAYOUT, ALIGN, ROWS)}))
        n = int(data.shape[0])
        admit((scale, Operand(kinds=(torch.float32,), count=n, dense=True),
               {**every(f"{f.name}: scale must be float32 with {n} values", KIND, EXTENT),
                LAYOUT: f"{f.name}: scale must be contiguous"}))  # fmt: skip
        if off_card(self.index, data, scale, bias):
            raise ValueError(f"{f.name}: the weight's tensors must be on cuda:{self.index}")
        self._half(out_dtype)
        if bias is not None and bias.numel() != n:
            raise ValueError(f"{f.name}: bias must have {n} values")
        return None if bias is None else _aligned(bias.to(out_dtype))

    # -------------------------------------------------------------- LoRA bake

    def bake(self, form: int, data: Tensor, scale: Tensor | None, up: Tensor, down: Tensor,
             seed: int, *, gain: Tensor | None = None, more: Tensor | None = None,
             flags: int = 0, rescale: Tensor | None = None) -> None:  # fmt: skip
        """`cozyq_bake` in place (`_bake_kernel`, `internal/lora_bake.py:1013-1053`): `data`
        contiguous [rows, cols] of the form, `scale` float32 [rows] (row-scaled forms), `up`
        float32 [rows, rank], `down` float32 [rank, cols] (int8.convrot: rotated). `gain`
        (float32 [rows], plain forms), `more` (float32 [rows, cols]) and `flags` (1 nearest,
        2 no delta) are the eager bake's additions; `rescale` (float32 [rows], fp8.rowwise) bakes
        onto new row scales, which the caller then stores."""
        rows, cols = (int(v) for v in data.shape)
        stored = (data,) if scale is None else (data, scale)
        rank = self._factors(up, down, rows, cols, stored, gain, more)
        if rescale is not None and (rescale.dtype != self.torch.float32 or rescale.numel() != rows
                                    or not rescale.is_contiguous()):  # fmt: skip
            raise ValueError(f"LoRA bake: new row scales must be contiguous float32 with {rows} values")
        code = self._lib.cozyq_bake(
            self.index, form, data.data_ptr(), _ptr(scale), up.data_ptr(), down.data_ptr(),
            _ptr(gain), _ptr(more), _ptr(rescale), rows, cols, rank, seed & 0xFFFFFFFF, flags,
            self._stream(),
        )  # fmt: skip
        self._check(code, "the LoRA bake")

    def bake_nvfp4_refit(self, data: Tensor, blocks: Tensor, second: Tensor, up: Tensor, down: Tensor,
                         seed: int, level: float, *, flags: int = 0, gain: Tensor | None = None,
                         more: Tensor | None = None) -> None:  # fmt: skip
        """`cozyq_bake_nvfp4_refit` in place (`bake_nvfp4` with `grid="refit"`,
        `internal/lora_bake.py:458-525`): decodes at `second` (times `gain` per row), adds
        `up @ down` (and `more`), refits every block on the new second level `level` (a float64
        the caller then stores), `flags` 1 for nearest."""
        rows, cols = int(data.shape[0]), 2 * int(data.shape[1])
        if tuple(blocks.shape) != (rows, cols // 16) or not blocks.is_contiguous():
            raise ValueError(f"nvfp4 bake: block scales must be contiguous [{rows}, {cols // 16}]")
        rank = self._factors(up, down, rows, cols, (data, blocks, second), gain, more)
        code = self._lib.cozyq_bake_nvfp4_refit(
            self.index, data.data_ptr(), blocks.data_ptr(), second.data_ptr(), float(level), up.data_ptr(),
            down.data_ptr(), _ptr(gain), _ptr(more), rows, cols, rank, seed & 0xFFFFFFFF, flags, self._stream(),
        )  # fmt: skip
        self._check(code, "the nvfp4 refit LoRA bake")

    def bake_feedback(self, data: Tensor, scale: Tensor, up: Tensor, down: Tensor, fresh: Tensor,
                      more: Tensor | None = None) -> None:  # fmt: skip
        """`cozyq_bake_feedback` in place (`encode_e4m3` with `feedback` under `bake_rowwise`,
        `internal/lora_bake.py:163-197`, `:319-363`): `data` contiguous E4M3 [rows, cols],
        `scale` its float32 row scales, `fresh` float32 [rows] the scales after the bake (the
        same values for `keep`), `more` LoKr's dense rows added to the delta; every 32-column run
        carries its nearest-rounding error."""
        rows, cols = (int(v) for v in data.shape)
        rank = self._factors(up, down, rows, cols, (data, scale), None, more)
        if fresh.dtype != self.torch.float32 or fresh.numel() != rows or not fresh.is_contiguous():
            raise ValueError(f"LoRA bake: new row scales must be contiguous float32 with {rows} values")
        code = self._lib.cozyq_bake_feedback(
            self.index, data.data_ptr(), scale.data_ptr(), fresh.data_ptr(), up.data_ptr(),
            down.data_ptr(), _ptr(more), rows, cols, rank, self._stream(),
        )  # fmt: skip
        self._check(code, "the error-feedback LoRA bake")

    def bake_nvfp4(self, data: Tensor, blocks: Tensor, second: Tensor, up: Tensor, down: Tensor,
                   seed: int, *, gain: Tensor | None = None, more: Tensor | None = None,
                   flags: int = 0) -> None:  # fmt: skip
        """`cozyq_bake_nvfp4` in place (`_bake_nvfp4_kernel`, `internal/lora_bake.py:955-1011`):
        codes uint8 [rows, cols/2], E4M3 block bytes uint8 [rows, cols/16], float32 `second`;
        `gain`, `more` and `flags` as `bake`'s (the eager `bake_nvfp4`, `:458-525`)."""
        rows, cols = int(data.shape[0]), 2 * int(data.shape[1])
        if tuple(blocks.shape) != (rows, cols // 16) or not blocks.is_contiguous():
            raise ValueError(f"nvfp4 bake: block scales must be contiguous [{rows}, {cols // 16}]")
        rank = self._factors(up, down, rows, cols, (data, blocks, second), gain, more)
        code = self._lib.cozyq_bake_nvfp4(
            self.index, data.data_ptr(), blocks.data_ptr(), second.data_ptr(), up.data_ptr(),
            down.data_ptr(), _ptr(gain), _ptr(more), rows, cols, rank, seed & 0xFFFFFFFF, flags,
            self._stream(),
        )  # fmt: skip
        self._check(code, "the nvfp4 LoRA bake")

    def bake_norms(self, form: int, data: Tensor, scale: Tensor | None, up: Tensor, down: Tensor,
                   *, cols: int, blocks: Tensor | None = None, second: Tensor | None = None,
                   amax: bool = False, gain: Tensor | None = None,
                   more: Tensor | None = None) -> Tensor:  # fmt: skip
        """`cozyq_bake_norms` (`norms`, `internal/lora_bake.py:653-689`): each row's L2 norm of
        the decoded weight plus `up @ down`, float32 [rows]; with `amax`, `cozyq_bake_row_amax`
        (each row's max |·|, the decoded rows times `gain` and LoKr's `more` added if given).
        form 5 is nvfp4 (codes `data`, `blocks`, `second`)."""
        rows = int(data.shape[0])
        if not amax and (gain is not None or more is not None):
            raise ValueError("bake_norms: a gain or dense rows enter the row maxima only")
        stored = tuple(t for t in (data, scale, blocks, second) if t is not None)
        rank = self._factors(up, down, rows, cols, stored, gain, more)
        out = self.torch.empty(rows, dtype=self.torch.float32, device=data.device)
        if amax:
            code = self._lib.cozyq_bake_row_amax(
                self.index, form, data.data_ptr(), _ptr(scale), _ptr(blocks), _ptr(second),
                up.data_ptr(), down.data_ptr(), _ptr(gain), _ptr(more), rows, cols, rank,
                out.data_ptr(), self._stream(),
            )  # fmt: skip
        else:
            code = self._lib.cozyq_bake_norms(
                self.index, form, data.data_ptr(), _ptr(scale), _ptr(blocks), _ptr(second),
                up.data_ptr(), down.data_ptr(), rows, cols, rank, out.data_ptr(), self._stream(),
            )  # fmt: skip
        self._check(code, "the row reduction")
        return out

    def bake_stats(self, form: int, before: dict[str, Tensor], after: dict[str, Tensor], up: Tensor,
                   down: Tensor, *, cols: int, gain: Tensor | None = None,
                   more: Tensor | None = None) -> Tensor:  # fmt: skip
        """`cozyq_bake_stats` (`_account`, `internal/lora_bake.py:249-268`): the accounting of one
        bake from its parts before and after (`data`, and `scale` or `blocks` + `second`; nvfp4's
        `before["second"]`, if given, is the level the stored weight decoded at before a refit),
        float64 [groups, 7] partial sums."""
        data = after["data"]
        rows = int(data.shape[0])
        rank = self._factors(up, down, rows, cols, tuple(after.values()) + tuple(before.values()), gain, more)
        partial = self.torch.empty((rows + 63) // 64, 7, dtype=self.torch.float64, device=data.device)
        code = self._lib.cozyq_bake_stats(
            self.index, form, before["data"].data_ptr(), data.data_ptr(), _ptr(before.get("scale")),
            _ptr(after.get("scale")), _ptr(before.get("blocks")), _ptr(after.get("blocks")),
            _ptr(before.get("second", after.get("second"))), _ptr(after.get("second")), _ptr(gain), _ptr(more),
            up.data_ptr(), down.data_ptr(), rows, cols, rank, partial.data_ptr(), self._stream(),
        )  # fmt: skip
        self._check(code, "the bake accounting")
        return partial

    def rotate_factor(self, down: Tensor) -> Tensor:
        """`cozyq_bake_rotate_factor` (`rotate_factor`, `internal/lora_bake.py:366-369`): float32
        [rank, cols] times H256/16 per 256 columns, into a new tensor."""
        if down.dtype != self.torch.float32 or down.dim() != 2 or not down.is_contiguous():
            raise ValueError("rotate_factor: down must be contiguous float32 [rank, cols]")
        if down.get_device() != self.index:
            raise ValueError(f"rotate_factor: down must be on cuda:{self.index}")
        out = self.torch.empty_like(down)
        code = self._lib.cozyq_bake_rotate_factor(
            self.index, down.data_ptr(), out.data_ptr(), int(down.shape[0]), int(down.shape[1]),
            self._stream(),
        )  # fmt: skip
        self._check(code, "the factor rotation")
        return out

    def _factors(self, up: Tensor, down: Tensor, rows: int, cols: int, stored: tuple,
                 gain: Tensor | None = None, more: Tensor | None = None) -> int:  # fmt: skip
        torch = self.torch
        for t in (up, down):
            if t.dtype != torch.float32 or t.dim() != 2 or not t.is_contiguous():
                raise ValueError("LoRA bake: factors must be contiguous float32 matrices")
        if gain is not None and (gain.dtype != torch.float32 or gain.numel() != rows
                                 or not gain.is_contiguous()):  # fmt: skip
            raise ValueError(f"LoRA bake: gain must be contiguous float32 with {rows} values")
        if more is not None and (more.dtype != torch.float32 or tuple(more.shape) != (rows, cols)
                                 or not more.is_contiguous()):  # fmt: skip
            raise ValueError(f"LoRA bake: dense rows must be contiguous float32 [{rows}, {cols}]")
        stored = stored + tuple(t for t in (gain, more) if t is not None)
        rank = int(up.shape[1])
        if int(up.shape[0]) != rows or tuple(down.shape) != (rank, cols):
            raise ValueError(f"LoRA bake: up must be [{rows}, rank] and down [rank, {cols}]; got "
                             f"{tuple(up.shape)} and {tuple(down.shape)}")  # fmt: skip
        for t in (*stored, up, down):
            if not t.is_cuda or t.get_device() != self.index:
                raise ValueError(f"LoRA bake: every tensor must be on cuda:{self.index}")
        if not stored[0].is_contiguous():
            raise ValueError("a fused bake writes a contiguous [out, in] weight")
        return rank

    def _half(self, dtype: Dtype) -> bool:
        """Contract V4: the kernels' flag for a 16-bit activation or output dtype (fp16 True,
        bf16 False); any other dtype raises."""
        half = self._halves.get(dtype)
        if half is None:
            raise ValueError(f"8-bit linear: activations and outputs are bf16 or fp16, not {dtype}")
        return half

    def _stream(self) -> int:
        """The raw handle of torch's current stream on this card, which every launch uses."""
        return int(self.torch.cuda.current_stream(self.index).cuda_stream)

    def _check(self, code: int, what: str) -> None:
        """`internal/prebuilt.py:428-434`."""
        if code == 0:
            return
        detail = f"8-bit linear: {what}: {_lib.error_name(code)}"
        if code == self._lib.cozyq_out_of_memory():
            raise self.torch.cuda.OutOfMemoryError(detail)
        raise RuntimeError(detail)


def _out_type(torch: Any, dtype: Dtype) -> int:
    """The decode kernels' destination code: 0 f32, 1 bf16, 2 f16."""
    return {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[dtype]


def _landed(result: Tensor, out: Tensor | None) -> Tensor:
    if out is None or result is out:
        return result
    out.copy_(result)
    return out


_LIBRARIES: dict[int, Prebuilt] = {}


def library(index: int = 0) -> Prebuilt:
    """The op library on cuda:`index`, opened once and only once each format's kernels pass their
    self-check on the card (`internal/prebuilt.py:568-598`; `cozyq.verify`). Raises
    `_lib.KernelsAbsent` where the HIP library is not built or loadable, and RuntimeError where
    the device is not the gfx950 the library carries or a format fails its check."""
    found = _LIBRARIES.get(index)
    if found is not None:
        return found
    torch = _torch()
    if not torch.cuda.is_available():
        raise RuntimeError("cozyq: no GPU visible")
    arch = torch.cuda.get_device_properties(index).gcnArchName.split(":")[0]
    carried = _lib.load().cozyq_arch().decode()
    if arch != carried:
        raise RuntimeError(f"cozyq carries {carried} device code; cuda:{index} is {arch}")
    ops = Prebuilt(torch, index)
    digest = verify.library_digest(_lib.PATH)
    with torch.cuda.device(index):
        ops.verdicts = {
            name: verify.verified(f"{name}-{arch}-{digest}", partial(probe, torch, ops),
                                  verify.cuda_fault(torch))
            for name, probe in verify.PROBES.items()
        }  # fmt: skip
    failed = [f"{name}: {v.detail}" for name, v in ops.verdicts.items() if not v.ok]
    if failed:
        raise RuntimeError(f"cozyq: the kernels failed their self-check on cuda:{index} ({arch}): "
                           + "; ".join(failed))
    _LIBRARIES[index] = ops
    return ops

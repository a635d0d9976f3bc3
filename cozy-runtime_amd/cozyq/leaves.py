"""Encoded-GEMM leaves on gfx950 — cozyq's counterpart of cozy-runtime's
`internal/encoding/leaves.py` (`EncodedLinear`, `NativeLinear`, the `*NativeLeaf` providers)
and of its launch table (`internal/encoding/selection.py:248-274`).

A provider (`LeafProvider`, `internal/encoding/formats.py:326-361`) turns one stored scheme's
parts into a leaf: an `nn.Module` standing where the replaced linear stood, whose weight is
its role buffers and whose forward is one of the gfx950 ops. Names, schemes, role names,
`BUFFERS`, `WRITES_INTO`, `operand`, `forward(x, *, prequantized=None, out=None)` and the
autocast behaviour are the reference's; the device predicate names the gfx950 row, and the
W4A4 provider serves this build's int4-g64 SVDQuant scheme in place of the reference's nvfp4.
"""

from __future__ import annotations

import functools
from collections.abc import Mapping, Sequence
from dataclasses import dataclass
from typing import Any, ClassVar

from cozyq import decode as dec
from cozyq import fp8_linear, int8_linear, layout, nvfp4_linear, prebuilt, w4a8_linear
from cozyq.operands import INT8_CONVROT, ROWWISE_FP8, PreQuantized, read, shared_operand

Tensor = Any
Dtype = Any
Params = tuple[tuple[str, object], ...]

MXFP8 = "cozy.mxfp8.native-leaf/2"
W4A8 = "cozy.w4a8-convrot256.native-leaf/1"
SVDQ_INT4 = "cozyq.svdq-int4g64.native-leaf/1"
NVFP4 = "cozy.nvfp4.native-leaf/1"
#: The operand geometry each 8-bit leaf's GEMM reads (`internal/encoding/leaves.py:207`).
OPERANDS = {INT8_CONVROT: INT8_CONVROT, ROWWISE_FP8: ROWWISE_FP8, W4A8: INT8_CONVROT}
#: The 8-bit leaves' ops by provider (`internal/encoding/leaves.py:355`).
_NATIVE_OPS: dict[str, Any] = {INT8_CONVROT: int8_linear, ROWWISE_FP8: fp8_linear}
#: Rows a leaf sends to its op's one-launch linear instead of a shared operand: the int8 GEMV
#: rows (the reference's `few`), and for fp8 the fused quantize + GEMV kernel's.
_FEW_ROWS = {INT8_CONVROT: int8_linear.GEMV_ROWS, ROWWISE_FP8: 4}
#: The card rows (the reference keys them by CUDA capability, `arch.py:51-64`): the
#: tensor-core formats each multiplies in.
ARCH_ROWS = {"gfx950": frozenset({"int8", "fp8", "mxfp8", "int4", "bf16"})}
DEVICE_PREDICATE = "rocm.gfx950"
INT8_ROTATION = 256
MX_BLOCK = 32
SVDQ_GROUP = 64
SVDQ_RANKS = (16, 32, 64)


def _rank2(shape: Sequence[int]) -> str:
    return "" if len(shape) == 2 else f"an encoded GEMM takes a rank-2 weight; this one is {list(shape)}"


def _leaf_geometry(replaced: object, data: Tensor) -> tuple[int, int, Tensor | None]:
    """`(in_features, out_features, bias)` of the module stood in for
    (`internal/encoding/leaves.py:437-448`)."""
    out_features, in_features = int(data.shape[0]), int(data.shape[1])
    return in_features, out_features, getattr(replaced, "bias", None)


def _leaf_class(torch: Any) -> Any:
    """`EncodedLinear`, built once, lazily (`internal/encoding/leaves.py:234-355`): the roles
    are buffers (never Parameters), registered under `BUFFERS`' names."""
    cached = getattr(_leaf_class, "_cached", None)
    if cached is not None:
        return cached
    from torch import nn

    class EncodedLinear(nn.Module):
        """One linear whose weight is its encoded role set, computed by an encoded GEMM."""

        BUFFERS: ClassVar[dict[str, str]] = {}
        WRITES_INTO: ClassVar[bool] = False
        PURE_WINDOWS: ClassVar[bool] = True

        def __init__(self, forward_fn, roles: Mapping[str, Tensor], bias: Tensor | None,
                     out_dtype: Dtype, provider: str, encoding: str, in_features: int,
                     out_features: int) -> None:  # fmt: skip
            super().__init__()
            # The replaced projection's compute dtype, for code that reads the first floating
            # buffer before casting activations; no bytes, not persisted.
            self.register_buffer("_logical_dtype",
                                 next(iter(roles.values())).new_empty(0, dtype=out_dtype),
                                 persistent=False)  # fmt: skip
            self._cozy_forward = forward_fn
            self._cozy_roles = tuple(sorted(roles))
            for role, tensor in sorted(roles.items()):
                self.register_buffer(self.BUFFERS.get(role, role), tensor)
            self.register_buffer("bias", bias)
            self.out_dtype = out_dtype
            self.provider = provider
            self.encoding = encoding
            self.in_features = in_features
            self.out_features = out_features

        def roles(self) -> dict[str, Tensor]:
            return {role: getattr(self, self.BUFFERS.get(role, role)) for role in self._cozy_roles}

        def forward(self, x: Tensor, *, prequantized: PreQuantized | None = None,
                    out: Tensor | None = None) -> Tensor:  # fmt: skip
            """The linear; with `out` (e.g. this linear's column range of a sibling group's
            packed output) the result lands there, which it also returns."""
            if out is None:
                return self.linear(x, prequantized)
            if self.WRITES_INTO:
                return self.linear(x, prequantized, out)
            out.copy_(self.linear(x, prequantized))
            return out

        def linear(self, x: Tensor, prequantized: PreQuantized | None,
                   out: Tensor | None = None) -> Tensor:  # fmt: skip
            forward = self._cozy_forward
            assert forward is not None  # a leaf built without one overrides `linear`
            if prequantized is None and torch.is_autocast_enabled(x.device.type):
                dtype = torch.get_autocast_dtype(x.device.type)
                result = forward(self, x.to(dtype), dtype)
            else:
                result = forward(self, x if prequantized is None else prequantized, self.out_dtype)
            if self.bias is not None:
                result = result + self.bias.to(result.dtype)
            return result

        def extra_repr(self) -> str:
            return (f"in_features={self.in_features}, out_features={self.out_features}, "
                    f"provider={self.provider!r}, roles={list(self._cozy_roles)}, "
                    f"out_dtype={self.out_dtype}")  # fmt: skip

    _leaf_class._cached = EncodedLinear
    return EncodedLinear


def _native_leaf_class(torch: Any) -> Any:
    """`NativeLinear` (`internal/encoding/leaves.py:358-434`): the forward is one call of its
    provider's op, the bias in the GEMM's epilogue, and a shared operand where siblings read
    the same input."""
    cached = getattr(_native_leaf_class, "_cached", None)
    if cached is not None:
        return cached

    class NativeLinear(_leaf_class(torch)):
        BUFFERS: ClassVar[dict[str, str]] = {"weight": "data"}
        WRITES_INTO: ClassVar[bool] = True

        @property
        def operand(self) -> str:
            return OPERANDS[self.provider]

        def linear(self, x, prequantized, out=None):
            ops = _NATIVE_OPS[self.provider]
            out_dtype = self.out_dtype
            data, scale, bias = read(self.data), read(self.scale), read(self.bias)
            if isinstance(x, PreQuantized):
                # A producer's prologue (`int8_rows`) hands the operand in place of x.
                if torch.is_autocast_enabled(x.payload.device.type):
                    out_dtype = torch.get_autocast_dtype(x.payload.device.type)
                return ops.gemm(torch, x, data, scale, bias, out_dtype, out)
            cast = x
            if torch.is_autocast_enabled(x.device.type):
                out_dtype = torch.get_autocast_dtype(x.device.type)
                cast = x.to(out_dtype)
            few = x.numel() <= _FEW_ROWS[self.provider] * x.shape[-1]
            if prequantized is None and few:
                # A decode step's few rows: the op's one-launch linear.
                return int8_linear.landed(ops.linear(torch, cast, data, scale, bias, out_dtype), out)
            if prequantized is None or prequantized.provider != self.provider:
                capturing = x.is_cuda and torch.cuda.is_current_stream_capturing()
                sibling = None if capturing else self
                prequantized = shared_operand(x, self.provider, lambda: ops.quantize(torch, cast),
                                              sibling)  # fmt: skip
            if prequantized is not None:
                return ops.gemm(torch, prequantized, data, scale, bias, out_dtype, out)
            return int8_linear.landed(ops.linear(torch, cast, data, scale, bias, out_dtype), out)

        def int8_prologue(self, x, consumers, norm, eps, scale, shift, activation, up=None):
            """`int8_rows` for consumers led by this leaf."""
            return int8_linear.prologue(torch, x, consumers, norm=norm, eps=eps, scale=scale,
                                        shift=shift, activation=activation, up=up)  # fmt: skip

    _native_leaf_class._cached = NativeLinear
    return NativeLinear


def _w4a8_leaf_class(torch: Any) -> Any:
    """`NativeLinear` over w4a8's roles (`internal/encoding/leaves.py:900-942`): its GEMM
    (`w4a8_linear`) on int8.convrot's operand, shared with the int8 leaves."""
    cached = getattr(_w4a8_leaf_class, "_cached", None)
    if cached is not None:
        return cached

    class W4a8Linear(_native_leaf_class(torch)):
        def weights(self) -> prebuilt.W4a8:
            return prebuilt.W4a8(read(self.data), read(self.group_scale), read(self.scale),
                                 read(self._buffers.get("codebook")))  # fmt: skip

        def linear(self, x, prequantized, out=None):
            out_dtype = self.out_dtype
            if isinstance(x, PreQuantized):
                if torch.is_autocast_enabled(x.payload.device.type):
                    out_dtype = torch.get_autocast_dtype(x.payload.device.type)
                return w4a8_linear.gemm(torch, x, self.weights(), read(self.bias), out_dtype, out)
            cast = x
            if torch.is_autocast_enabled(x.device.type):
                out_dtype = torch.get_autocast_dtype(x.device.type)
                cast = x.to(out_dtype)
            if prequantized is None or prequantized.provider != INT8_CONVROT:
                capturing = x.is_cuda and torch.cuda.is_current_stream_capturing()
                sibling = None if capturing else self
                prequantized = shared_operand(x, INT8_CONVROT,
                                              lambda: int8_linear.quantize(torch, cast), sibling)  # fmt: skip
            if prequantized is not None:
                return w4a8_linear.gemm(torch, prequantized, self.weights(), read(self.bias),
                                        out_dtype, out)  # fmt: skip
            return int8_linear.landed(
                w4a8_linear.linear(torch, cast, self.weights(), read(self.bias), out_dtype), out)

    _w4a8_leaf_class._cached = W4a8Linear
    return W4a8Linear


def _svdq_leaf_class(torch: Any) -> Any:
    """The W4A4 leaf: smoothing, int4 activations and the low-rank input in one launch, then
    the GEMM with the low-rank add and the bias in its epilogue (one rounding)."""
    cached = getattr(_svdq_leaf_class, "_cached", None)
    if cached is not None:
        return cached

    class SvdqLinear(_leaf_class(torch)):
        def linear(self, x, prequantized, out=None):
            if prequantized is not None:
                raise ValueError("the svdq leaf quantizes its own input; it takes no shared operand")
            out_dtype = self.out_dtype
            if torch.is_autocast_enabled(x.device.type):
                out_dtype = torch.get_autocast_dtype(x.device.type)
                x = x.to(out_dtype)
            int8_linear._served(torch, x, out_dtype)
            lib = int8_linear.library(x.get_device())
            result = lib.svdq_linear(x, read(self.pre_quant_scale), read(self.lowrank_down),
                                     read(self.weight), read(self.scale), read(self.lowrank_up),
                                     read(self.bias), out_dtype)  # fmt: skip
            return int8_linear.landed(result, out)

    _svdq_leaf_class._cached = SvdqLinear
    return SvdqLinear


def _mx_forward(torch: Any, leaf: Any, x: Tensor, out_dtype: Dtype) -> Tensor:
    """`MicroScaledNativeLeaf._forward` (`internal/encoding/leaves.py:1505-1516`): the
    activation quantized per 32-block at dispatch, the scaled-MFMA GEMM; the bias is added by
    `EncodedLinear.linear` after the cast, as the reference's is."""
    int8_linear._served(torch, x, out_dtype)
    lib = int8_linear.library(x.get_device())
    out = lib.mx_linear(x, leaf.weight, leaf.scale, None, out_dtype)
    return out.reshape(*x.shape[:-1], -1)


class _Provider:
    """The `LeafProvider` members every encoded-GEMM provider here answers alike."""

    @property
    def route(self) -> str:
        return "encoded_gemm"

    @property
    def device_predicate(self) -> str:
        return DEVICE_PREDICATE

    @property
    def output_dtype_rule(self) -> str:
        return "contract"

    @property
    def out_dtypes(self) -> frozenset[str]:
        return frozenset({"bfloat16", "float16"})

    @property
    def optional(self) -> frozenset[str]:
        return frozenset()

    def decode(self, torch: Any, parts: Mapping[str, Tensor], destination: Tensor) -> None:
        raise AssertionError("an encoded_gemm provider replaces the leaf; it never writes a float "
                             "destination — see LeafProvider.leaf")  # fmt: skip

    def resident_bytes(self, parts: Mapping[str, Any]) -> int:
        return sum(int(p.nbytes) for p in parts.values())

    def resident_bits_per_element(self, parts: Mapping[str, Any], numel: int) -> float:
        return 8.0 * self.resident_bytes(parts) / max(numel, 1)

    def fill_scratch_bytes(self, parts: Mapping[str, Any]) -> int:
        return 0


@dataclass(frozen=True, slots=True)
class RowwiseNativeLeaf(_Provider):
    """fp8.rowwise encoded GEMM (`internal/encoding/leaves.py:451-551`): W8A8 e4m3, per-token
    activation scales at dispatch, per-output-row weight scales, float32 accumulation."""

    encoding: str = "fp8.rowwise"
    params: Params = ()

    name = property(lambda self: ROWWISE_FP8)
    schemes = property(lambda self: frozenset({"fp8.rowwise"}))
    code_revision = property(lambda self: "1")
    suite = property(lambda self: "fp8-rowwise-native")
    formats = property(lambda self: frozenset({"fp8"}))
    required = property(lambda self: frozenset({"weight", "scale"}))

    def supports(self, shape: Sequence[int], params: Mapping[str, object]) -> str:
        """Rank 2, 16-byte rows (K % 16) and N % 8 for the fp8 GEMM's epilogue."""
        why = _rank2(shape)
        if why or (int(shape[1]) % 16 == 0 and int(shape[0]) % 8 == 0):
            return why
        return f"the fp8 GEMM needs K divisible by 16 and N by 8; this tensor is {list(shape)}"

    def leaf(self, torch: Any, parts: Mapping[str, Tensor], replaced: object, out_dtype: Dtype) -> Any:
        data = parts["weight"]
        in_features, out_features, bias = _leaf_geometry(replaced, data)
        return _native_leaf_class(torch)(
            None, {"weight": data, "scale": parts["scale"].to(torch.float32)}, bias, out_dtype,
            self.name, self.encoding, in_features, out_features)  # fmt: skip


@dataclass(frozen=True, slots=True)
class Int8ConvRotNativeLeaf(_Provider):
    """int8-convrot256 encoded GEMM (`internal/encoding/leaves.py:554-656`): weight rows rotated
    by the regular Hadamard per 256 input channels offline, activation rows rotated and
    quantized per token at dispatch, W8A8 on the int8 MFMA with exact int32 accumulation."""

    encoding: str = "int8.convrot"
    params: Params = ()

    name = property(lambda self: INT8_CONVROT)
    schemes = property(lambda self: frozenset({"int8.convrot"}))
    code_revision = property(lambda self: "1")
    suite = property(lambda self: "int8-convrot256-native")
    formats = property(lambda self: frozenset({"int8"}))
    required = property(lambda self: frozenset({"weight", "scale"}))

    def supports(self, shape: Sequence[int], params: Mapping[str, object]) -> str:
        """Rank 2, 256-groups (the rotation), N % 8."""
        why = _rank2(shape)
        if not why and params.get("rotation_size") != INT8_ROTATION:
            why = (f"the int8 kernel rotates {INT8_ROTATION}-groups; this weight's are "
                   f"{params.get('rotation_size')}")  # fmt: skip
        if not why and int(shape[1]) % INT8_ROTATION:
            why = f"the int8 kernel rotates whole {INT8_ROTATION}-groups; this tensor is {list(shape)}"
        if why or int(shape[0]) % 8 == 0:
            return why
        return f"the int8 GEMM needs N divisible by 8 and this tensor has {shape[0]} rows"

    def leaf(self, torch: Any, parts: Mapping[str, Tensor], replaced: object, out_dtype: Dtype) -> Any:
        data = parts["weight"]
        in_features, out_features, bias = _leaf_geometry(replaced, data)
        return _native_leaf_class(torch)(
            None, {"weight": data, "scale": parts["scale"].to(torch.float32)}, bias, out_dtype,
            self.name, self.encoding, in_features, out_features)  # fmt: skip


@dataclass(frozen=True, slots=True)
class W4a8NativeLeaf(_Provider):
    """`w4a8.convrot` encoded GEMM (`internal/encoding/leaves.py:945-1045`): 4-bit codes in
    int8.convrot's rotated basis with E4M3 group scales per 16 and a row scale (4.5 bits a
    weight), unpacked to int8 levels in registers and multiplied with int8.convrot's operand
    on the int8 MFMA: W4A8 with int8.convrot's epilogue. It takes group 16, rotation 256, and a
    codebook or the uniform grid."""

    encoding: str = "w4a8.convrot"
    params: Params = ()

    name = property(lambda self: W4A8)
    schemes = property(lambda self: frozenset({"w4a8.convrot"}))
    code_revision = property(lambda self: "1")
    suite = property(lambda self: "w4a8-native")
    formats = property(lambda self: frozenset({"int8"}))
    required = property(lambda self: frozenset({"weight", "group_scale", "scale"}))
    optional = property(lambda self: frozenset({"codebook"}))

    def supports(self, shape: Sequence[int], params: Mapping[str, object]) -> str:
        """Rank 2; group 16 and int8.convrot's 256-blocks; N divisible by 8."""
        why = _rank2(shape)
        wanted = {"group_size": 16, "rotation": "kron_regular_h4", "rotation_size": INT8_ROTATION}
        if not why and dict(params) != wanted:
            why = f"the w4a8 GEMM reads {wanted}; this weight's are {dict(params)}"
        if not why and (int(shape[1]) % INT8_ROTATION or int(shape[0]) % 8):
            why = f"the w4a8 GEMM needs K % {INT8_ROTATION} and N % 8 == 0; this is {list(shape)}"
        return why

    def leaf(self, torch: Any, parts: Mapping[str, Tensor], replaced: object, out_dtype: Dtype) -> Any:
        codes = parts["weight"]
        roles = {"weight": codes, "group_scale": parts["group_scale"],
                 "scale": parts["scale"].to(torch.float32)}  # fmt: skip
        if "codebook" in parts:
            roles["codebook"] = parts["codebook"].to(torch.float32)
        return _w4a8_leaf_class(torch)(None, roles, getattr(replaced, "bias", None), out_dtype,
                                       self.name, self.encoding, 2 * int(codes.shape[1]),
                                       int(codes.shape[0]))  # fmt: skip


@dataclass(frozen=True, slots=True)
class MicroScaledNativeLeaf(_Provider):
    """mxfp8 encoded GEMM (`internal/encoding/leaves.py:1427-1546`) on gfx950's E8M0-scaled
    MFMA: the e4m3 payload and its E8M0 grid stay resident; activations are quantized per
    32-block at dispatch. The grid is kept row-major `[N, K/32]` (the kernel's layout): a part
    stored in cuBLAS's 128x4 tiles is untiled once, at fill."""

    encoding: str = "mxfp8"
    params: Params = ()

    name = property(lambda self: MXFP8)
    schemes = property(lambda self: frozenset({"mxfp8"}))
    code_revision = property(lambda self: "2")
    suite = property(lambda self: "mxfp8-native")
    formats = property(lambda self: frozenset({"mxfp8"}))
    required = property(lambda self: frozenset({"weight", "scale"}))

    def supports(self, shape: Sequence[int], params: Mapping[str, object]) -> str:
        """Rank 2, whole 128-element K steps of the scaled MFMA, N % 8."""
        why = _rank2(shape)
        if why:
            return why
        if int(shape[1]) % 128 or int(shape[0]) % 8:
            return f"the MX GEMM reads 128-element K steps and N % 8 == 0; this tensor is {list(shape)}"
        return ""

    def resident_bytes(self, parts: Mapping[str, Any]) -> int:
        rows, cols = int(parts["weight"].shape[0]), int(parts["weight"].shape[1]) // MX_BLOCK
        return int(parts["weight"].nbytes) + rows * cols

    def fill_scratch_bytes(self, parts: Mapping[str, Any]) -> int:
        rows, cols = int(parts["weight"].shape[0]), int(parts["weight"].shape[1]) // MX_BLOCK
        return 2 * rows * cols  # the untiled grid and its index table's bytes

    def leaf(self, torch: Any, parts: Mapping[str, Tensor], replaced: object, out_dtype: Dtype) -> Any:
        weight = parts["weight"]
        if weight.dtype != torch.float8_e4m3fn:
            raise ValueError(f"the MX GEMM takes E4M3 weights and this one is {weight.dtype}")
        in_features, out_features, bias = _leaf_geometry(replaced, weight)
        rows, cols = int(weight.shape[0]), int(weight.shape[1]) // MX_BLOCK
        scale = parts["scale"].view(torch.uint8)
        if dict(self.params).get("scale_layout") == "cublas_128x4":
            scale = layout.from_blocked(torch, scale, rows, cols)
        else:
            scale = scale.reshape(rows, cols).contiguous()
        return _leaf_class(torch)(
            functools.partial(_mx_forward, torch), {"weight": weight, "scale": scale}, bias,
            out_dtype, self.name, self.encoding, in_features, out_features)  # fmt: skip


@dataclass(frozen=True, slots=True)
class SvdqInt4NativeLeaf(_Provider):
    """SVDQuant W4A4, int4-g64 (this build's scheme; the reference's SvdqNvfp4NativeLeaf,
    `internal/encoding/leaves.py:1266-1390`, serves nvfp4): residual codes packed two a byte
    with fp16 scales per 64-group, a per-input-channel smoothing vector, and the bf16 low-rank
    branch `bf16(x·downᵀ)·upᵀ`, added in the GEMM's epilogue."""

    encoding: str = "svdq.int4g64"
    params: Params = ()

    name = property(lambda self: SVDQ_INT4)
    schemes = property(lambda self: frozenset({"svdq.int4g64"}))
    code_revision = property(lambda self: "1")
    suite = property(lambda self: "svdq-int4g64-native")
    formats = property(lambda self: frozenset({"int4"}))
    required = property(lambda self: frozenset(
        {"weight", "scale", "pre_quant_scale", "lowrank_down", "lowrank_up"}))

    def supports(self, shape: Sequence[int], params: Mapping[str, object]) -> str:
        """Rank 2 (`[N, K/2]` packed bytes), whole 64-groups, N % 8, a served rank."""
        why = _rank2(shape)
        if why:
            return why
        k = 2 * int(shape[1])
        if k % SVDQ_GROUP or int(shape[0]) % 8:
            return f"the svdq GEMM needs K % {SVDQ_GROUP} == 0 and N % 8 == 0; this tensor is {list(shape)}"
        rank = params.get("rank")
        if rank is not None and rank not in SVDQ_RANKS:
            return f"the svdq kernels take ranks {SVDQ_RANKS}, not {rank}"
        return ""

    def leaf(self, torch: Any, parts: Mapping[str, Tensor], replaced: object, out_dtype: Dtype) -> Any:
        weight = parts["weight"]
        out_features, in_features = int(weight.shape[0]), 2 * int(weight.shape[1])
        roles = {
            "weight": weight.view(torch.uint8),
            "scale": parts["scale"].to(torch.float16),
            "pre_quant_scale": parts["pre_quant_scale"].to(torch.float32),
            "lowrank_down": parts["lowrank_down"].to(torch.bfloat16),
            "lowrank_up": parts["lowrank_up"].to(torch.bfloat16),
        }
        return _svdq_leaf_class(torch)(None, roles, getattr(replaced, "bias", None), out_dtype,
                                       self.name, self.encoding, in_features, out_features)  # fmt: skip


def _nvfp4_leaf_class(torch: Any) -> Any:
    """`EncodedLinear` keyed by nvfp4's stored roles (`internal/encoding/leaves.py:1056-1065`)."""
    cached = getattr(_nvfp4_leaf_class, "_cached", None)
    if cached is not None:
        return cached

    class Nvfp4Linear(_leaf_class(torch)):  # type: ignore[misc]
        BUFFERS: ClassVar[dict[str, str]] = {"scale": "weight_scale", "scale_2": "weight_scale_2"}

    _nvfp4_leaf_class._cached = Nvfp4Linear
    return Nvfp4Linear


def _nvfp4_forward(torch: Any, leaf: Any, x: Tensor, out_dtype: Dtype) -> Tensor:
    """`Nvfp4NativeLeaf._forward` (`internal/encoding/leaves.py:1158-1170`)."""
    return nvfp4_linear.matmul(torch, x, leaf.weight, leaf.weight_scale, None, leaf.weight_scale_2,
                               out_dtype)  # fmt: skip


@dataclass(frozen=True, slots=True)
class Nvfp4NativeLeaf(_Provider):
    """`nvfp4` encoded GEMM (`internal/encoding/leaves.py:1069-1203`): the E2M1 payload and E4M3
    block scales stay resident (0.56 bytes a weight). Up to 16 rows take the W4A16 GEMV on the
    bf16/fp16 MFMA; more rows decode the weight per 128-row chunk and take the library GEMM. The
    scales are held in cuBLAS's 128x4 tiles and the nibbles low first, as the reference's leaf
    holds them; a `divide` second level is held as its float32 reciprocal, as there."""

    encoding: str = "nvfp4"
    params: Params = ()

    name = property(lambda self: NVFP4)
    schemes = property(lambda self: frozenset({"nvfp4"}))
    code_revision = property(lambda self: "1")
    suite = property(lambda self: "nvfp4-native")
    # The reference's leaf names none (W4A16 runs on every MMA card); here the kernels multiply on
    # gfx950's bf16/fp16 MFMA.
    formats = property(lambda self: frozenset({"bf16"}))
    out_dtypes = property(lambda self: frozenset({"bfloat16", "float16", "float32"}))
    required = property(lambda self: frozenset({"weight", "scale", "scale_2"}))
    optional = property(lambda self: frozenset({"input_scale"}))

    def supports(self, shape: Sequence[int], params: Mapping[str, object]) -> str:
        """The decode's block law, and K % 32, N % 8 (`internal/encoding/leaves.py:1127-1134`)."""
        why = _rank2(shape) or dec.Nvfp4Dequant().supports(shape, params)
        if why:
            return why
        if int(shape[1]) % 32 or int(shape[0]) % 8:
            return f"the FP4 GEMM needs K % 32 == 0 and N % 8 == 0; this tensor is {list(shape)}"
        return ""

    def resident_bytes(self, parts: Mapping[str, Any]) -> int:
        rows, cols = dec.blocked_shape(int(parts["scale"].shape[0]), int(parts["scale"].shape[1]))
        return int(parts["weight"].nbytes) + rows * cols + 4

    def fill_scratch_bytes(self, parts: Mapping[str, Any]) -> int:
        rows, cols = dec.blocked_shape(int(parts["scale"].shape[0]), int(parts["scale"].shape[1]))
        return 3 * rows * cols

    def leaf(self, torch: Any, parts: Mapping[str, Tensor], replaced: object, out_dtype: Dtype) -> Any:
        params = dict(self.params)
        weight = parts["weight"].view(torch.uint8)
        if params.get("nibble_order") == "high_first":
            weight = (weight << 4) | (weight >> 4)  # the kernels read element 2k low
        out_features, in_features = int(weight.shape[0]), 2 * int(weight.shape[1])
        rows, cols = dec.blocked_shape(out_features, in_features // 16)
        if params.get("scale_layout") == "cublas_128x4":
            blocked = parts["scale"].view(torch.uint8).reshape(rows, cols)
        else:
            blocked = layout.to_blocked(torch, parts["scale"].view(torch.uint8).reshape(
                out_features, in_features // 16)).view(rows, cols)  # fmt: skip
        second = parts["scale_2"].to(torch.float32).reshape(1)
        if params.get("global_scale") == "divide":
            second = 1.0 / second
        return _nvfp4_leaf_class(torch)(
            functools.partial(_nvfp4_forward, torch),
            {"weight": weight, "scale": blocked.view(torch.float8_e4m3fn), "scale_2": second},
            getattr(replaced, "bias", None), out_dtype, self.name, self.encoding, in_features,
            out_features)  # fmt: skip


def launch_providers() -> dict[str, tuple[Any, ...]]:
    """Scheme -> its encoded-GEMM providers on gfx950, in the reference's preference order
    (`internal/encoding/selection.py:248-274`, the encoded_gemm entries)."""
    out: dict[str, list[Any]] = {}
    for build in (RowwiseNativeLeaf, Int8ConvRotNativeLeaf, W4a8NativeLeaf, SvdqInt4NativeLeaf,
                  MicroScaledNativeLeaf, Nvfp4NativeLeaf):
        for scheme in sorted(build().schemes):
            out.setdefault(scheme, []).append(build(scheme))
    return {scheme: tuple(candidates) for scheme, candidates in out.items()}


def serves(provider: Any, arch: str) -> bool:
    """Whether a card of `arch` multiplies in every format the provider's kernels use."""
    return provider.formats <= ARCH_ROWS.get(arch, frozenset())

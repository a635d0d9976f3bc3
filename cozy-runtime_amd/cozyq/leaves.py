"""Encoded-GEMM leaves on gfx950 — cozyq's counterpart of cozy-runtime's
`internal/encoding/leaves.py` (`EncodedLinear`, `NativeLinear`, the `*NativeLeaf` providers)
and of its launch table (`internal/encoding/selection.py:248-274`).

A provider (`LeafProvider`, `internal/encoding/formats.py:326-361`) turns one stored scheme's
parts into a leaf: an `nn.Module` standing where the replaced linear stood, whose weight is
its role buffers and whose forward is one of the gfx950 ops. Names, schemes, role names,
`BUFFERS`, `WRITES_INTO`, `operand`, `forward(x, *, prequantized=None, out=None)` and the
autocast behaviour are the reference's; the device predicate names the gfx950 row. The W4A4
providers serve the reference's svdq.nvfp4 scheme and this build's int4-g64 SVDQuant variant.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping, Sequence
from dataclasses import dataclass
from typing import Any, ClassVar

from cozyq import _dispatch, fp8_linear, int8_linear, layout, nvfp4_linear, prebuilt, svdq_linear, w4a8_linear
from cozyq import decode as dec
from cozyq.operands import INT8_CONVROT, ROWWISE_FP8, PreQuantized, read, shared_operand

Tensor = Any
Dtype = Any
Params = tuple[tuple[str, object], ...]

MXFP8 = "cozy.mxfp8.native-leaf/2"
W4A8 = "cozy.w4a8-convrot256.native-leaf/1"
SVDQ_INT4 = "cozyq.svdq-int4g64.native-leaf/1"
SVDQ = "cozy.svdq-nvfp4.native-leaf/1"
NVFP4 = "cozy.nvfp4.native-leaf/1"
#: The operand geometry each 8-bit leaf's GEMM reads (`internal/encoding/leaves.py:207`).
OPERANDS = {INT8_CONVROT: INT8_CONVROT, ROWWISE_FP8: ROWWISE_FP8, W4A8: INT8_CONVROT}
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
    """`(in_features, out_features, bias)`: the features from the stored `[N, K]` weight, the
    bias from the module stood in for (`internal/encoding/leaves.py:437-448`)."""
    return int(data.shape[1]), int(data.shape[0]), getattr(replaced, "bias", None)


def _autocast_dtype(torch: Any, device: Any) -> Dtype | None:
    kind = device.type
    return torch.get_autocast_dtype(kind) if torch.is_autocast_enabled(kind) else None


# ----------------------------------------------------------------------------- lanes
#
# A lane is how one family of leaves computes: the buffer names of its roles, whether its GEMM
# writes the caller's `out`, the operand geometry it reads, and `run`. The module class below is
# the same for every family and holds its lane.


class _Lane:
    buffers: Mapping[str, str] = {}
    writes_into = False
    operand: str | None = None

    def run(self, torch: Any, leaf: Any, x: Any, prequantized: PreQuantized | None,
            out: Tensor | None) -> Tensor:  # fmt: skip
        raise NotImplementedError


class _FloatLane(_Lane):
    """Leaves that compute from the 16-bit activation and add the bias afterwards, in the
    result's dtype (rules L3, L5): the MX and nvfp4 leaves. `compute(torch, leaf, x, out_dtype)`
    is the product."""

    def __init__(self, compute: Callable[..., Tensor], buffers: Mapping[str, str] | None = None) -> None:
        self.compute = compute
        self.buffers = dict(buffers or {})

    def run(self, torch, leaf, x, prequantized, out):
        if prequantized is not None or isinstance(x, PreQuantized):
            raise ValueError(f"{leaf.provider} computes from the activation; it takes no quantized operand")
        dtype = _autocast_dtype(torch, x.device)
        product = self.compute(torch, leaf, x if dtype is None else x.to(dtype),
                               leaf.out_dtype if dtype is None else dtype)  # fmt: skip
        return product if leaf.bias is None else product + leaf.bias.to(product.dtype)


class _QuantizedLane(_Lane):
    """The 8-bit leaves (rule L4): a producer's operand goes straight to the GEMM; up to
    `few` rows with no operand take the op's one-launch linear; otherwise the operand handed
    in (if it has this lane's geometry) or one shared with the sibling leaves, else the
    one-call linear. The bias is in the GEMM's epilogue; the GEMM writes `out`."""

    buffers = {"weight": "data"}
    writes_into = True

    def __init__(self, operand: str, few: int) -> None:
        self.operand = operand
        self.few = few

    # The op calls, per family.
    def quantize(self, torch: Any, x: Tensor) -> PreQuantized | None:
        return int8_linear.quantize(torch, x)

    def gemm(self, torch, leaf, operand, out_dtype, out):
        return int8_linear.gemm(torch, operand, read(leaf.data), read(leaf.scale), read(leaf.bias),
                                out_dtype, out)  # fmt: skip

    def linear(self, torch, leaf, x, out_dtype):
        return int8_linear.linear(torch, x, read(leaf.data), read(leaf.scale), read(leaf.bias), out_dtype)

    def run(self, torch, leaf, x, prequantized, out):
        if isinstance(x, PreQuantized):
            dtype = _autocast_dtype(torch, x.payload.device)
            return self.gemm(torch, leaf, x, leaf.out_dtype if dtype is None else dtype, out)
        dtype = _autocast_dtype(torch, x.device)
        x16, out_dtype = (x, leaf.out_dtype) if dtype is None else (x.to(dtype), dtype)
        operand = prequantized if prequantized is not None and prequantized.provider == self.operand else None
        if operand is None:
            if prequantized is None and x.numel() <= self.few * x.shape[-1]:
                return _dispatch.deliver(self.linear(torch, leaf, x16, out_dtype), out)
            capturing = x.is_cuda and torch.cuda.is_current_stream_capturing()
            operand = shared_operand(x, self.operand, lambda: self.quantize(torch, x16),
                                     None if capturing else leaf)  # fmt: skip
        if operand is None:
            return _dispatch.deliver(self.linear(torch, leaf, x16, out_dtype), out)
        return self.gemm(torch, leaf, operand, out_dtype, out)


class _Fp8Lane(_QuantizedLane):
    def quantize(self, torch, x):
        return fp8_linear.quantize(torch, x)

    def gemm(self, torch, leaf, operand, out_dtype, out):
        return fp8_linear.gemm(torch, operand, read(leaf.data), read(leaf.scale), read(leaf.bias),
                               out_dtype, out)  # fmt: skip

    def linear(self, torch, leaf, x, out_dtype):
        return fp8_linear.linear(torch, x, read(leaf.data), read(leaf.scale), read(leaf.bias), out_dtype)


class _W4a8Lane(_QuantizedLane):
    """w4a8 codes on int8.convrot's operand: the int8 lane's quantize, its own GEMM."""

    @staticmethod
    def _weights(leaf: Any) -> prebuilt.W4a8:
        return prebuilt.W4a8(read(leaf.data), read(leaf.group_scale), read(leaf.scale),
                             read(leaf._buffers.get("codebook")))  # fmt: skip

    def gemm(self, torch, leaf, operand, out_dtype, out):
        return w4a8_linear.gemm(torch, operand, self._weights(leaf), read(leaf.bias), out_dtype, out)

    def linear(self, torch, leaf, x, out_dtype):
        return w4a8_linear.linear(torch, x, self._weights(leaf), read(leaf.bias), out_dtype)


class _SvdqLane(_Lane):
    """The W4A4 leaf: smoothing, int4 activation codes and the low-rank input in one launch,
    then the GEMM with the low-rank term and the bias before its one rounding."""

    def run(self, torch, leaf, x, prequantized, out):
        if prequantized is not None or isinstance(x, PreQuantized):
            raise ValueError("the svdq leaf quantizes its own input; it takes no shared operand")
        dtype = _autocast_dtype(torch, x.device)
        out_dtype = leaf.out_dtype if dtype is None else dtype
        x = x if dtype is None else x.to(dtype)
        index = _dispatch.activation_card("svdq", torch, x, out_dtype)
        result = _dispatch.library(index).svdq_int4_linear(
            x, read(leaf.pre_quant_scale), read(leaf.lowrank_down), read(leaf.weight),
            read(leaf.scale), read(leaf.lowrank_up), read(leaf.bias), out_dtype)  # fmt: skip
        return result


class _SvdqNvfp4Lane(_Lane):
    """The svdq.nvfp4 leaf (`internal/encoding/leaves.py:1205-1263`): the activation smoothed,
    quantized and down-projected in one launch, then the GEMM with the up-projection, c and the
    bias before its one rounding. A baked request's LoRAs (`adopt`) enter the branch as more ranks
    while the ranks together fit the kernels' largest, else as their own term afterwards."""

    adopts = True

    def run(self, torch, leaf, x, prequantized, out):
        if prequantized is not None or isinstance(x, PreQuantized):
            raise ValueError("the svdq leaf quantizes its own input; it takes no shared operand")
        dtype = _autocast_dtype(torch, x.device)
        out_dtype = leaf.out_dtype if dtype is None else dtype
        x = x if dtype is None else x.to(dtype)
        roles = {role: read(t) for role, t in leaf.roles().items()}
        deltas = leaf.lora() if leaf.lora is not None else []
        apart = None
        if deltas:
            bound = [read(t) for d in deltas for t in d[1:3]]
            key = (roles["lowrank_down"].data_ptr(), roles["lowrank_up"].data_ptr(),
                   *((d[0], d[3]) for d in deltas), *(t.data_ptr() for t in bound))  # fmt: skip
            cached = leaf._cozy_merged
            if cached is None or cached[0] != key:
                down = torch.cat(bound[0::2])
                up = torch.cat([u * d[3] for u, d in zip(bound[1::2], deltas, strict=True)], dim=1)
                cached = (key, svdq_linear.merged(torch, roles, down, up), (down, up))
                leaf._cozy_merged = cached
            if cached[1] is not None:
                roles.update(cached[1])
            else:
                apart = cached[2]
        y = svdq_linear.linear(torch, x, roles, read(leaf.bias), out_dtype)
        if apart is not None:  # more ranks than the kernels take: the LoRAs' own term
            down, up = apart
            y = y + ((x.to(down.dtype) @ down.t()) @ up.t()).to(y.dtype)
        return y


def _mx_product(torch: Any, leaf: Any, x: Tensor, out_dtype: Dtype) -> Tensor:
    """The MX leaf's product (`internal/encoding/leaves.py:1505-1516`): x quantized per 32-block
    at dispatch, then the scaled-MFMA GEMM; the lane adds the bias after the cast."""
    index = _dispatch.activation_card("mxfp8", torch, x, out_dtype)
    return _dispatch.library(index).mx_linear(x, leaf.weight, leaf.scale, None, out_dtype).reshape(
        *x.shape[:-1], -1)  # fmt: skip


def _nvfp4_product(torch: Any, leaf: Any, x: Tensor, out_dtype: Dtype) -> Tensor:
    """The nvfp4 leaf's product (`internal/encoding/leaves.py:1158-1170`)."""
    return nvfp4_linear.matmul(torch, x, leaf.weight, leaf.weight_scale, None, leaf.weight_scale_2,
                               out_dtype)  # fmt: skip


_NVFP4_BUFFERS = {"scale": "weight_scale", "scale_2": "weight_scale_2"}


def _module_class(torch: Any) -> Any:
    """The `nn.Module` every encoded leaf is (built once, on first use): rules L1–L2, the rest
    delegated to the leaf's lane."""
    cached = getattr(_module_class, "_cached", None)
    if cached is not None:
        return cached

    class EncodedLinear(torch.nn.Module):
        """A linear whose weight is its encoded role buffers; `forward` runs its lane."""

        PURE_WINDOWS: ClassVar[bool] = True

        def __init__(self, lane: _Lane, roles: Mapping[str, Tensor], bias: Tensor | None,
                     out_dtype: Dtype, provider: str, encoding: str, in_features: int,
                     out_features: int) -> None:  # fmt: skip
            super().__init__()
            self._cozy_lane = lane
            self._cozy_roles = tuple(sorted(roles))
            device = next(iter(roles.values())).device
            self.register_buffer("_logical_dtype", torch.empty(0, dtype=out_dtype, device=device),
                                 persistent=False)  # fmt: skip
            for role in self._cozy_roles:
                self.register_buffer(lane.buffers.get(role, role), roles[role])
            self.register_buffer("bias", bias)
            self.out_dtype = out_dtype
            self.provider, self.encoding = provider, encoding
            self.in_features, self.out_features = in_features, out_features

        @property
        def BUFFERS(self) -> dict[str, str]:  # noqa: N802 (the reference's attribute name)
            return dict(self._cozy_lane.buffers)

        @property
        def WRITES_INTO(self) -> bool:  # noqa: N802
            return self._cozy_lane.writes_into

        @property
        def operand(self) -> str | None:
            """The activation geometry this leaf's GEMM reads (8-bit leaves), else None."""
            return self._cozy_lane.operand

        #: A baked request's LoRAs (the reference's `SvdqLinear.lora`): what returns each one's
        #: `(identity, down [r, K], up [N, r], scale)` as the forward runs; None for none. Only a
        #: lane that `adopts` reads it.
        lora: Callable[[], list[tuple[object, Tensor, Tensor, float]]] | None = None
        #: The branch with the LoRAs merged in, for the factors bound at these addresses.
        _cozy_merged: tuple[tuple[object, ...], dict[str, Tensor] | None, tuple[Tensor, Tensor]] | None = None

        def adopt(self, lora: Callable[[], list[tuple[object, Tensor, Tensor, float]]] | None) -> None:
            """Binds a baked request's LoRAs (`internal/encoding/leaves.py:1223-1226`)."""
            if not getattr(self._cozy_lane, "adopts", False):
                raise TypeError(f"{self.provider} leaves take no LoRA branch")
            self.lora = lora

        def roles(self) -> dict[str, Tensor]:
            names = self._cozy_lane.buffers
            return {role: getattr(self, names.get(role, role)) for role in self._cozy_roles}

        def forward(self, x: Any, *, prequantized: PreQuantized | None = None,
                    out: Tensor | None = None) -> Tensor:  # fmt: skip
            lane = self._cozy_lane
            result = lane.run(torch, self, x, prequantized, out if lane.writes_into else None)
            if out is None or result is out:
                return result
            out.copy_(result)
            return out

        def int8_prologue(self, x, consumers, norm, eps, scale, shift, activation, up=None):
            """`int8_rows` for consumers led by this leaf (int8.convrot's operand)."""
            return int8_linear.prologue(torch, x, consumers, norm=norm, eps=eps, scale=scale,
                                        shift=shift, activation=activation, up=up)  # fmt: skip

        def extra_repr(self) -> str:
            return ", ".join((f"in_features={self.in_features}", f"out_features={self.out_features}",
                              f"provider={self.provider!r}", f"roles={list(self._cozy_roles)}",
                              f"out_dtype={self.out_dtype}"))  # fmt: skip

    _module_class._cached = EncodedLinear
    return EncodedLinear


def _build(torch: Any, lane: _Lane, roles: Mapping[str, Tensor], bias: Tensor | None,
           out_dtype: Dtype, provider: Any, in_features: int, out_features: int) -> Any:  # fmt: skip
    return _module_class(torch)(lane, roles, bias, out_dtype, provider.name, provider.encoding,
                                in_features, out_features)  # fmt: skip


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
        return _build(torch, _Fp8Lane(ROWWISE_FP8, _FEW_ROWS[ROWWISE_FP8]),
                      {"weight": data, "scale": parts["scale"].to(torch.float32)}, bias, out_dtype,
                      self, in_features, out_features)  # fmt: skip


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
        return _build(torch, _QuantizedLane(INT8_CONVROT, _FEW_ROWS[INT8_CONVROT]),
                      {"weight": data, "scale": parts["scale"].to(torch.float32)}, bias, out_dtype,
                      self, in_features, out_features)  # fmt: skip


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
        return _build(torch, _W4a8Lane(INT8_CONVROT, _FEW_ROWS[INT8_CONVROT]), roles,
                      getattr(replaced, "bias", None), out_dtype, self, 2 * int(codes.shape[1]),
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
        return _build(torch, _FloatLane(_mx_product), {"weight": weight, "scale": scale}, bias,
                      out_dtype, self, in_features, out_features)  # fmt: skip


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
        return _build(torch, _SvdqLane(), roles, getattr(replaced, "bias", None), out_dtype, self,
                      in_features, out_features)  # fmt: skip


@dataclass(frozen=True, slots=True)
class SvdqNvfp4NativeLeaf(_Provider):
    """`svdq.nvfp4` encoded GEMM (`internal/encoding/leaves.py:1267-1407`): SVDQuant's nvfp4
    residual, its smoothing and its 16-bit low-rank branch stay resident and are multiplied as
    they are (`svdq_linear`): the activation is smoothed, quantized to nvfp4 and down-projected in
    one pass, and the GEMM decodes both operands exactly onto the matrix core and adds the
    up-projection in its epilogue. The weight is held as stored (row-major scales, element 2k
    low); a high-first nibble order, cuBLAS scale tiles, a divided second level, an unbuilt rank
    and 16-bit factors other than bf16 are converted once, at the bind."""

    encoding: str = "svdq.nvfp4"
    params: Params = ()

    name = property(lambda self: SVDQ)
    schemes = property(lambda self: frozenset({"svdq.nvfp4"}))
    code_revision = property(lambda self: "1")
    suite = property(lambda self: "svdq-nvfp4-native")
    # The reference's kernels multiply on FP4 tensor cores; these on gfx950's fp16/bf16 MFMA.
    formats = property(lambda self: frozenset({"bf16"}))
    required = property(lambda self: frozenset(
        {"weight", "scale", "scale_2", "pre_quant_scale", "lowrank_down", "lowrank_up"}))
    optional = property(lambda self: frozenset({"input_scale", "channel_scale"}))

    def supports(self, shape: Sequence[int], params: Mapping[str, object]) -> str:
        """One matrix, nvfp4's block law, K whole GEMM steps and N % 8
        (`internal/encoding/leaves.py:1322-1330`, with this GEMM's own multiples)."""
        why = _rank2(shape) or dec.Nvfp4Dequant().supports(shape, params)
        if not why and (int(shape[1]) % svdq_linear.K_ALIGN or int(shape[0]) % 8):
            why = (f"the svdq GEMM needs K % {svdq_linear.K_ALIGN} == 0 and N % 8 == 0; this tensor "
                   f"is {list(shape)}")  # fmt: skip
        return why

    def leaf(self, torch: Any, parts: Mapping[str, Tensor], replaced: object, out_dtype: Dtype) -> Any:
        """`internal/encoding/leaves.py:1347-1407`: the roles where the kernels read them."""
        params = dict(self.params)
        down, up = parts["lowrank_down"], parts["lowrank_up"]
        if int(down.shape[0]) > svdq_linear.RANKS[-1]:
            raise ValueError(f"a rank-{int(down.shape[0])} branch: the svdq kernels take up to "
                             f"{svdq_linear.RANKS[-1]}; it decodes instead")  # fmt: skip
        weight = parts["weight"].view(torch.uint8)
        if params.get("nibble_order") == "high_first":
            weight = (weight << 4) | (weight >> 4)  # the kernels read element 2k low
        out_features, in_features = int(weight.shape[0]), 2 * int(weight.shape[1])
        scale = parts["scale"].view(torch.uint8)
        if params.get("scale_layout") == "cublas_128x4":
            scale = layout.from_blocked(torch, scale, out_features, in_features // 16)
        scale = scale.reshape(out_features, in_features // 16).contiguous().view(torch.float8_e4m3fn)
        second = parts["scale_2"].to(torch.float32).reshape(1)
        if params.get("global_scale") == "divide":
            second = 1.0 / second
        rank = int(down.shape[0])
        if svdq_linear.rank(rank) != rank or torch.bfloat16 not in (down.dtype, up.dtype):
            down, up = svdq_linear.padded(torch, down, up)
        elif down.dtype != up.dtype:
            down, up = down.to(torch.bfloat16), up.to(torch.bfloat16)
        roles = {"weight": weight.contiguous(), "scale": scale, "scale_2": second,
                 "pre_quant_scale": parts["pre_quant_scale"].to(torch.float32).reshape(-1),
                 "lowrank_down": down.contiguous(), "lowrank_up": up.contiguous()}  # fmt: skip
        for role in ("channel_scale", "input_scale"):
            if role in parts:
                roles[role] = parts[role].to(torch.float32).reshape(-1)
        return _build(torch, _SvdqNvfp4Lane(), roles, getattr(replaced, "bias", None), out_dtype,
                      self, in_features, out_features)  # fmt: skip


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
        return _build(torch, _FloatLane(_nvfp4_product, _NVFP4_BUFFERS),
                      {"weight": weight, "scale": blocked.view(torch.float8_e4m3fn), "scale_2": second},
                      getattr(replaced, "bias", None), out_dtype, self, in_features, out_features)  # fmt: skip


def launch_providers() -> dict[str, tuple[Any, ...]]:
    """Scheme -> its encoded-GEMM providers on gfx950, in the reference's preference order
    (`internal/encoding/selection.py:248-274`, the encoded_gemm entries)."""
    out: dict[str, list[Any]] = {}
    for build in (RowwiseNativeLeaf, Int8ConvRotNativeLeaf, W4a8NativeLeaf, SvdqNvfp4NativeLeaf,
                  SvdqInt4NativeLeaf, MicroScaledNativeLeaf, Nvfp4NativeLeaf):
        for scheme in sorted(build().schemes):
            out.setdefault(scheme, []).append(build(scheme))
    return {scheme: tuple(candidates) for scheme, candidates in out.items()}


def serves(provider: Any, arch: str) -> bool:
    """Whether a card of `arch` multiplies in every format the provider's kernels use."""
    return provider.formats <= ARCH_ROWS.get(arch, frozenset())

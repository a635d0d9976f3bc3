"""Stored-format decode providers on gfx950: cozyq's stand-ins for cozy-runtime's
`decoded_float` providers, which turn a checkpoint's encoded parts into a float weight.

- `TensorwiseDequant`, `RowwiseDequant` (+ `columnwise`), `MicroScaledDequant`,
  `Int8ConvRotDequant`, `Nvfp4Dequant` ↔ `internal/encoding/formats.py:438-868`.
- `CoreDequant` for `nvfp4` and `svdq.nvfp4` ↔ `internal/encoding/adapters.py:33-102` over the
  rows of `internal/decode_schemes.py:340-500`.

Each keeps the reference's name, route, schemes, roles, params rule and `supports` messages.
`decode(torch, parts, destination)` writes the destination with one HIP kernel (`cozyq_decode`,
`cozyq_decode_convrot`, `cozyq_decode_svdq`): the same float32 steps as the reference's chunked
torch ops, one rounding into the destination. The reference decodes on any device; these decode
on the GPU only, and parts or a destination off it raise ValueError.

`part_rule` is the fill plane's check of a stored tensor's parts (`formats.part_rule`,
`formats.py:193-238`, and `decode_schemes.parts_rule`, `decode_schemes.py:174-203`): what a
decode refuses before it runs.
"""

from __future__ import annotations

import math
from collections.abc import Mapping, Sequence
from dataclasses import dataclass
from typing import Any

Tensor = Any
Params = tuple[tuple[str, object], ...]

#: Destination dtypes a decode writes (`formats.py:114`).
DECODED = frozenset({"f32", "bf16", "f16"})
_F8 = frozenset({"f8_e4m3fn", "f8_e5m2"})
_SCALES = frozenset({"f32", "bf16", "f16"})
MX_BLOCK = 32
NVFP4_BLOCK = 16
SCALE_LAYOUTS = ("row_major", "cublas_128x4")
NIBBLE_ORDERS = ("low_first", "high_first")
GLOBAL_SCALES = ("multiply", "divide")
#: `int8.convrot`'s rotation sizes, `4**k` for 1 <= k <= 8 (`formats.py:655-656`).
ROTATION_SIZES = tuple(4**k for k in range(1, 9))
CONVROT_GROUP = 256

# The C ABI's codes (include/cozyq.h): element codes, part dtypes, scale grids.
_CODE = {"i8": 0, "f8_e4m3fn": 1, "f8_e5m2": 2, "u8": 3}
_NUM = {"f32": 0, "bf16": 1, "f16": 2, "f8_e8m0": 3, "u8": 3, "f8_e4m3fn": 4}
GRID_TENSOR, GRID_ROW, GRID_COL, GRID_BLOCKS = 0, 1, 2, 3

_NAMES = {
    "float32": "f32", "bfloat16": "bf16", "float16": "f16", "float8_e4m3fn": "f8_e4m3fn",
    "float8_e5m2": "f8_e5m2", "float8_e8m0fnu": "f8_e8m0", "uint8": "u8", "int8": "i8",
    "int16": "i16", "int32": "i32", "int64": "i64", "bool": "bool", "float64": "f64",
}  # fmt: skip


def dtype_name(dtype: Any) -> str:
    """A torch dtype's runtime name (`decode_schemes.TORCH`'s keys)."""
    return _NAMES.get(str(dtype).removeprefix("torch."), str(dtype))


def matrix(shape: Sequence[int]) -> tuple[int, int]:
    """`[rows, cols]`: the last axis, every leading axis a row (`formats.py:133-139`)."""
    rows = 1
    for extent in shape[:-1]:
        rows *= int(extent)
    return rows, int(shape[-1]) if shape else 0


def blocked_shape(rows: int, cols: int) -> tuple[int, int]:
    """cuBLAS's 128x4 tiled grid: rows up to 128s, columns up to 4s (`formats.py:153-154`)."""
    return -(-rows // 128) * 128, -(-cols // 4) * 4


# ---------------------------------------------------------------------------- part rules


def _params(params: Mapping[str, object], allowed: Mapping[str, Sequence[object]]) -> str:
    """`formats._params` (`formats.py:379-388`): exactly `allowed`'s keys, each allowed."""
    unknown = sorted(set(params) - set(allowed))
    if unknown:
        return f"unknown params {unknown}"
    for name, values in allowed.items():
        if params.get(name) not in values:
            return f"param {name}={params.get(name)!r}, expected one of {list(values)}"
    return ""


def _rows_rule(shape: Sequence[int]) -> str:
    """`formats._rows` (`formats.py:373-377`)."""
    if len(shape) < 2:
        return f"a row or block scheme needs two axes and this tensor is rank {len(shape)}"
    return ""


#: The row/tensor/convrot schemes' parts: role -> (dtypes, count or "shape")
#: (`formats.part_rule`, `formats.py:207-228`).
def _table_rules(scheme: str, shape: tuple[int, ...]) -> dict[str, tuple[frozenset[str], object]]:
    rows, cols = matrix(shape)
    i8 = frozenset({"i8"})
    one = frozenset({"f32"})
    return {
        "fp8.rowwise": {"weight": (_F8, shape), "scale": (_SCALES, rows)},
        "fp8.columnwise": {"weight": (_F8, shape), "scale": (_SCALES, cols)},
        "int8.rowwise": {"weight": (i8, shape), "scale": (_SCALES, rows)},
        "int8.columnwise": {"weight": (i8, shape), "scale": (_SCALES, cols)},
        "fp8.tensorwise": {"weight": (_F8, shape), "scale": (_SCALES, 1), "input_scale": (one, 1)},
        "int8.tensorwise": {"weight": (i8, shape), "scale": (_SCALES, 1), "input_scale": (one, 1)},
        "int8.convrot": {"weight": (i8, shape), "scale": (_SCALES, rows)},
    }.get(scheme, {})


@dataclass(frozen=True)
class _Row:
    """One core scheme's rule (`decode_schemes.Adapter`): params, parts and a cross rule."""

    scheme: str
    params: Mapping[str, tuple[object, ...]]
    required: frozenset[str]
    optional: frozenset[str]


_NVFP4_PARAMS = {
    "block_size": (NVFP4_BLOCK,), "global_scale": GLOBAL_SCALES, "nibble_order": NIBBLE_ORDERS,
    "scale_layout": SCALE_LAYOUTS,
}  # fmt: skip
CORE_ROWS = {
    "mxfp8": _Row("mxfp8", {"block_size": (MX_BLOCK,), "scale_layout": SCALE_LAYOUTS},
                  frozenset({"weight", "scale"}), frozenset()),
    "nvfp4": _Row("nvfp4", _NVFP4_PARAMS, frozenset({"weight", "scale", "scale_2"}),
                  frozenset({"input_scale", "pre_quant_scale"})),
    "svdq.nvfp4": _Row("svdq.nvfp4", _NVFP4_PARAMS,
                       frozenset({"weight", "scale", "scale_2", "pre_quant_scale", "lowrank_down",
                                  "lowrank_up"}),
                       frozenset({"input_scale", "channel_scale"})),
}  # fmt: skip


def _allowed(values: tuple[object, ...], value: object) -> bool:
    return any(type(value) is type(a) and value == a for a in values)


def _core_rule(
    row: _Row, shape: tuple[int, ...], params: Mapping[str, object],
    parts: Mapping[str, tuple[str, tuple[int, ...]]],
) -> str:
    """`decode_schemes.parts_rule` (`decode_schemes.py:174-203`) for the mxfp8, nvfp4 and
    svdq.nvfp4 rows (`:362-431,434-519,574-585`)."""
    s = row.scheme
    unknown = sorted(set(params) - set(row.params))
    if unknown:
        return f"{s}: unknown params {unknown}"
    for key, values in row.params.items():
        if key not in params:
            return f"{s}: param {key} is missing"
        if not _allowed(values, params[key]):
            return f"{s}: param {key}={params[key]!r}"
    if len(shape) < 2:
        return f"{s} views rank 2 or more, not {tuple(shape)}"
    if set(parts) - row.required - row.optional or row.required - set(parts):
        return f"{s}: parts {sorted(parts)}, requires {sorted(row.required)}"
    rows, cols = matrix(shape)
    lead, height, stack = shape[:-1], shape[-2], shape[:-2]
    matrices = math.prod(stack)
    block = MX_BLOCK if s == "mxfp8" else NVFP4_BLOCK
    width = -(-cols // block)
    if params["scale_layout"] == "cublas_128x4":
        grid = (*stack, *blocked_shape(height, width))
    else:
        grid = (*lead, width)

    def per_matrix(role: str) -> int:
        got = parts.get(role)
        return 1 if got is None or math.prod(got[1]) == 1 else matrices

    want: dict[str, tuple[tuple[str, ...], str, object]] = {}
    if s == "mxfp8":
        want["weight"] = (("f8_e4m3fn", "f8_e5m2"), "exact", tuple(shape))
        want["scale"] = (("f8_e8m0", "u8"), "exact", grid)
    else:
        if cols % 2:
            return f"{s}: F4 {list(shape)} is not whole bytes"
        want["weight"] = (("u8",), "exact", (*lead, cols // 2))
        want["scale"] = (("f8_e4m3fn",), "exact", grid)
        want["scale_2"] = (("f32",), "count", per_matrix("scale_2"))
        want["input_scale"] = (("f32",), "count", per_matrix("input_scale"))
        want["pre_quant_scale"] = (("f32", "bf16", "f16"), "count", cols)
    if s == "svdq.nvfp4":
        down, up = parts.get("lowrank_down"), parts.get("lowrank_up")
        for role, got, axis in (("lowrank_down", down, 0), ("lowrank_up", up, 1)):
            if got is not None and (len(got[1]) != 2 or got[1][axis] < 1):
                return f"{s}: {role} is not a rank-2 factor"
        rank_d = 32 if down is None else int(down[1][0])
        rank_u = 32 if up is None else int(up[1][1])
        want["channel_scale"] = (("f32", "f8_e4m3fn"), "count", rows)
        want["lowrank_down"] = (("bf16", "f16", "f32"), "exact", (rank_d, cols))
        want["lowrank_up"] = (("bf16", "f16", "f32"), "exact", (rows, rank_u))
    for role, (dtype, got) in parts.items():
        names, kind, extent = want[role]
        fits = tuple(got) == extent if kind == "exact" else math.prod(got) == extent
        if dtype not in names or not fits:
            return f"{s}: part {role} is {dtype} {list(got)}, wants {names} {kind} {extent}"
    if s == "svdq.nvfp4":
        if len(shape) != 2:
            return f"svdq.nvfp4 is one matrix, not {list(shape)}"
        if parts["lowrank_down"][1][0] != parts["lowrank_up"][1][-1]:
            return (f"svdq.nvfp4: lowrank_down {list(parts['lowrank_down'][1])} and lowrank_up "
                    f"{list(parts['lowrank_up'][1])} differ in rank")  # fmt: skip
    if s != "mxfp8" and cols % NVFP4_BLOCK:
        return f"{s}: {cols} columns are not whole blocks of 16"
    return ""


def part_rule(
    scheme: str, params: Mapping[str, object], shape: Sequence[int], dtype: str,
    parts: Mapping[str, tuple[str, Sequence[int]]],
) -> str:
    """"" when a stored tensor of `scheme` with these parts (runtime dtype name, shape) decodes
    into a `dtype` destination of `shape`, else why not (`formats.part_rule`,
    `formats.py:193-238`; the core rows' `decode_schemes.parts_rule`)."""
    shape = tuple(int(v) for v in shape)
    got = {role: (d, tuple(int(v) for v in s)) for role, (d, s) in parts.items()}
    if dtype not in DECODED:
        return f"{scheme} decodes to f32, bf16 or f16, not {dtype}"
    if scheme in CORE_ROWS:
        return _core_rule(CORE_ROWS[scheme], shape, params, got)
    provider = provider_for(scheme, params)
    if provider is None:
        return f"no decode provider serves {scheme}"
    why = provider.supports(shape, params)
    if why:
        return why
    if set(got) - provider.required - provider.optional or provider.required - set(got):
        return f"{scheme}: parts {sorted(got)}, requires {sorted(provider.required)}"
    for role, (names, want) in _table_rules(scheme, shape).items():
        part = got.get(role)
        if part is None:
            continue
        if part[0] not in names:
            return f"{scheme} part {role} is {part[0]}, not one of {sorted(names)}"
        extent: object = math.prod(part[1]) if isinstance(want, int) else part[1]
        if extent != want:
            return f"{scheme} part {role} has shape {list(part[1])}, expected {want}"
    return ""


# ------------------------------------------------------------------------------ helpers


def _ops(destination: Tensor) -> Any:
    """The op library on the destination's GPU; a destination off the GPU raises."""
    from cozyq.prebuilt import library

    if getattr(destination.device, "type", None) != "cuda":
        raise ValueError(f"cozyq decodes on the GPU; the destination is on {destination.device}")
    return library(destination.device.index or 0)


def _part(torch: Any, t: Tensor, destination: Tensor, align: int = 1) -> Tensor:
    """A part contiguous on the destination's device (at an `align`-byte address)."""
    if t.device != destination.device:
        raise ValueError(f"a part on {t.device} does not decode into {destination.device}")
    t = t.contiguous()
    return t if t.data_ptr() % align == 0 else t.clone()


def _num(t: Tensor) -> int:
    return _NUM[dtype_name(t.dtype)]


def _check_destination(destination: Tensor) -> None:
    if dtype_name(destination.dtype) not in DECODED or not destination.is_contiguous():
        raise ValueError(f"a decode writes a contiguous f32, bf16 or f16 tensor, not "
                         f"{destination.dtype}")  # fmt: skip


def _validate(scheme: str, params: Mapping[str, object], parts: Mapping[str, Tensor],
              destination: Tensor) -> None:
    why = part_rule(scheme, params, tuple(destination.shape), dtype_name(destination.dtype),
                    {r: (dtype_name(t.dtype), tuple(t.shape)) for r, t in parts.items()})
    if why:
        raise ValueError(why)


# ---------------------------------------------------------------------------- providers


@dataclass(frozen=True, slots=True)
class TensorwiseDequant:
    """`fp8.tensorwise` / `int8.tensorwise` -> float: `round(weight · scale)`
    (`formats.py:437-488`). `input_scale` never enters the weight."""

    encoding: str = "fp8.tensorwise"
    params: Params = ()

    @property
    def name(self) -> str:
        return {"int8.tensorwise": "cozy.int8-tensorwise.dequant/1"}.get(
            self.encoding, "cozy.fp8-tensorwise.dequant/1")

    route = property(lambda self: "decoded_float")
    device_predicate = property(lambda self: "rocm.gfx950")
    schemes = property(lambda self: frozenset({"fp8.tensorwise", "int8.tensorwise"}))
    code_revision = property(lambda self: "2")
    required = property(lambda self: frozenset({"weight", "scale"}))
    optional = property(lambda self: frozenset({"input_scale"}))

    @property
    def suite(self) -> str:
        return {"int8.tensorwise": "int8-tensorwise-decode"}.get(self.encoding,
                                                                 "fp8-tensorwise-decode")

    def supports(self, shape: Sequence[int], params: Mapping[str, object]) -> str:
        return _params(params, {})

    def decode(self, torch: Any, parts: Mapping[str, Tensor], destination: Tensor) -> None:
        _check_destination(destination)
        _validate(self.encoding, dict(self.params), parts, destination)
        ops = _ops(destination)
        rows, cols = matrix(destination.shape)
        weight = _part(torch, parts["weight"], destination)
        scale = _part(torch, parts["scale"], destination)
        ops.decode_table(_CODE[dtype_name(weight.dtype)], weight, scale, _num(scale),
                         destination, rows, cols, grid=GRID_TENSOR)  # fmt: skip


@dataclass(frozen=True, slots=True)
class RowwiseDequant:
    """`fp8.rowwise`, `int8.rowwise` and their `.columnwise` twins -> float: `weight[i, j] ·
    scale[i]` (or `scale[j]`) in float32, rounded once (`formats.py:506-575`)."""

    encoding: str = "fp8.rowwise"
    params: Params = ()

    @property
    def name(self) -> str:
        return {"fp8.rowwise": "cozy.fp8-rowwise.dequant/1"}.get(
            self.encoding, f"cozy.{self.encoding}.dequant/1")

    route = property(lambda self: "decoded_float")
    device_predicate = property(lambda self: "rocm.gfx950")
    code_revision = property(lambda self: "3")
    required = property(lambda self: frozenset({"weight", "scale"}))
    optional = property(lambda self: frozenset())

    @property
    def schemes(self) -> frozenset[str]:
        if self.encoding.endswith(".columnwise"):
            return frozenset({"fp8.columnwise", "int8.columnwise"})
        return frozenset({"fp8.rowwise", "int8.rowwise"})

    @property
    def suite(self) -> str:
        return self.encoding.replace(".", "-") + "-decode"

    def supports(self, shape: Sequence[int], params: Mapping[str, object]) -> str:
        why = _rows_rule(shape) or _params(params, {})
        if why or len(shape) == 2 or not self.encoding.endswith(".columnwise"):
            return why
        return "a per-column scale is a rank-2 weight's"

    def decode(self, torch: Any, parts: Mapping[str, Tensor], destination: Tensor) -> None:
        _check_destination(destination)
        _validate(self.encoding, dict(self.params), parts, destination)
        ops = _ops(destination)
        rows, cols = matrix(destination.shape)
        weight = _part(torch, parts["weight"], destination)
        scale = _part(torch, parts["scale"], destination)
        grid = GRID_COL if self.encoding.endswith(".columnwise") else GRID_ROW
        ops.decode_table(_CODE[dtype_name(weight.dtype)], weight, scale, _num(scale),
                         destination, rows, cols, grid=grid)  # fmt: skip


def columnwise(encoding: str = "") -> RowwiseDequant:
    """The columnwise dequant (`formats.py:572-575`)."""
    return RowwiseDequant(encoding or "fp8.columnwise")


@dataclass(frozen=True, slots=True)
class MicroScaledDequant:
    """`mxfp8` -> float: `weight[i, j] · 2**(scale[i, j // 32] - 127)` in float32 (exact),
    rounded once; a short last block decodes like any other (`formats.py:588-650`). Scale grids
    row-major or in cuBLAS's 128x4 tiles, read in place."""

    encoding: str = "mxfp8"
    params: Params = ()

    name = property(lambda self: "cozy.mxfp8.dequant/1")
    route = property(lambda self: "decoded_float")
    device_predicate = property(lambda self: "rocm.gfx950")
    schemes = property(lambda self: frozenset({"mxfp8"}))
    code_revision = property(lambda self: "2")
    suite = property(lambda self: "mxfp8-decode")
    required = property(lambda self: frozenset({"weight", "scale"}))
    optional = property(lambda self: frozenset())

    def supports(self, shape: Sequence[int], params: Mapping[str, object]) -> str:
        why = _rows_rule(shape) or _params(
            params, {"block_size": (MX_BLOCK,), "scale_layout": SCALE_LAYOUTS})
        if not why and len(shape) > 2 and params.get("scale_layout") == "cublas_128x4":
            return f"a tiled stack {tuple(shape)} decodes through the cores, one matrix at a time"
        return why

    def decode(self, torch: Any, parts: Mapping[str, Tensor], destination: Tensor) -> None:
        _decode_mx(torch, dict(self.params), parts, destination)


def _decode_mx(torch: Any, params: Mapping[str, object], parts: Mapping[str, Tensor],
               destination: Tensor) -> None:
    """The mxfp8 core row (`decode_schemes.py:516-585`): one matrix at a time under cuBLAS
    tiles, as one `[E·N, C]` matrix row-major."""
    _check_destination(destination)
    _validate("mxfp8", params, parts, destination)
    ops = _ops(destination)
    shape = tuple(destination.shape)
    cols = shape[-1]
    tiled = params["scale_layout"] == "cublas_128x4"
    matrices = math.prod(shape[:-2]) if tiled else 1
    rows = math.prod(shape[:-1]) // matrices
    weight = _part(torch, parts["weight"], destination, 16)
    scale = _part(torch, parts["scale"], destination)
    ops.decode_table(_CODE[dtype_name(weight.dtype)], weight, scale.view(torch.uint8),
                     _NUM["f8_e8m0"], destination, rows, cols, grid=GRID_BLOCKS, block=MX_BLOCK,
                     tiled=tiled, matrices=matrices)  # fmt: skip


@dataclass(frozen=True, slots=True)
class Int8ConvRotDequant:
    """`int8.convrot` -> float: `(y[i] · scale[i]) · 2^-k`, `y` the exact int32 Hadamard sum of
    each `rotation_size = 4^k` group of int8 weights, cast once (`formats.py:678-752`)."""

    encoding: str = "int8.convrot"
    params: Params = ()

    name = property(lambda self: "cozy.int8-convrot.dequant/1")
    route = property(lambda self: "decoded_float")
    device_predicate = property(lambda self: "rocm.gfx950")
    schemes = property(lambda self: frozenset({"int8.convrot"}))
    code_revision = property(lambda self: "1")
    suite = property(lambda self: "int8-convrot-decode")
    required = property(lambda self: frozenset({"weight", "scale"}))
    optional = property(lambda self: frozenset())

    def supports(self, shape: Sequence[int], params: Mapping[str, object]) -> str:
        why = _rows_rule(shape) or _params(
            params, {"rotation": ("kron_regular_h4",), "rotation_size": ROTATION_SIZES})
        size = int(str(params.get("rotation_size", 1)))
        if why or int(shape[-1]) % size == 0:
            return why
        return (f"int8.convrot rotates whole {size}-column groups; this tensor has {shape[-1]} "
                f"columns")  # fmt: skip

    def decode(self, torch: Any, parts: Mapping[str, Tensor], destination: Tensor) -> None:
        _check_destination(destination)
        _validate(self.encoding, dict(self.params), parts, destination)
        ops = _ops(destination)
        size = int(str(dict(self.params)["rotation_size"]))
        rows, cols = matrix(destination.shape)
        weight = _part(torch, parts["weight"], destination, 16)
        scale = _part(torch, parts["scale"], destination)
        target = destination if destination.data_ptr() % 16 == 0 else torch.empty_like(destination)
        ops.decode_convrot(weight, scale, _num(scale), size, target, rows, cols)
        if target is not destination:
            destination.copy_(target)


@dataclass(frozen=True, slots=True)
class Nvfp4Dequant:
    """`nvfp4` -> float: `(e2m1 · e4m3 scale) · scale_2`, or with `global_scale: divide`
    `e2m1 · (e4m3 scale ÷ scale_2)` (`formats.py:762-868`). `input_scale` is the activation's
    and never enters the weight."""

    encoding: str = "nvfp4"
    params: Params = ()

    name = property(lambda self: "cozy.nvfp4.dequant/1")
    route = property(lambda self: "decoded_float")
    device_predicate = property(lambda self: "rocm.gfx950")
    schemes = property(lambda self: frozenset({"nvfp4"}))
    code_revision = property(lambda self: "1")
    suite = property(lambda self: "nvfp4-decode")
    required = property(lambda self: frozenset({"weight", "scale", "scale_2"}))
    optional = property(lambda self: frozenset({"input_scale"}))

    def supports(self, shape: Sequence[int], params: Mapping[str, object]) -> str:
        why = _rows_rule(shape) or _params(params, _NVFP4_PARAMS)
        if why:
            return why
        if len(shape) > 2:
            return f"a stack {tuple(shape)} decodes through the cores, one matrix at a time"
        if int(shape[-1]) % NVFP4_BLOCK == 0:
            return ""
        return (f"nvfp4 scales whole {NVFP4_BLOCK}-column blocks; this tensor has {shape[-1]} "
                f"columns")  # fmt: skip

    def decode(self, torch: Any, parts: Mapping[str, Tensor], destination: Tensor) -> None:
        why = self.supports(tuple(destination.shape), dict(self.params))
        if why or "pre_quant_scale" in parts:
            raise ValueError(why or "nvfp4: the dequant provider takes no pre_quant_scale")
        _decode_nvfp4(torch, dict(self.params), parts, destination)


def _decode_nvfp4(torch: Any, params: Mapping[str, object], parts: Mapping[str, Tensor],
                  destination: Tensor) -> None:
    """The nvfp4 core row (`decode_schemes.py:362-431`): the table law, then `· pre_quant_scale`
    per column when given; a stack takes its own `scale_2` and, under cuBLAS tiles, its own
    scale grid."""
    _check_destination(destination)
    _validate("nvfp4", params, parts, destination)
    ops = _ops(destination)
    shape = tuple(destination.shape)
    cols, stack = shape[-1], math.prod(shape[:-2])
    second = _part(torch, parts["scale_2"], destination).reshape(-1).float()
    tiled = params["scale_layout"] == "cublas_128x4"
    matrices = stack if stack > 1 and (tiled or second.numel() > 1) else 1
    rows = math.prod(shape[:-1]) // matrices
    weight = _part(torch, parts["weight"], destination, 8)
    scale = _part(torch, parts["scale"], destination)
    post = parts.get("pre_quant_scale")
    post = None if post is None else _part(torch, post, destination)
    ops.decode_table(
        _CODE["u8"], weight.view(torch.uint8), scale.view(torch.uint8), _NUM["f8_e4m3fn"],
        destination, rows, cols, grid=GRID_BLOCKS, block=NVFP4_BLOCK, tiled=tiled,
        scale_2=second, per_matrix=second.numel() > 1, divide=params["global_scale"] == "divide",
        post=post, post_type=0 if post is None else _num(post),
        high_first=params["nibble_order"] == "high_first", matrices=matrices,
    )  # fmt: skip


def _decode_svdq(torch: Any, params: Mapping[str, object], parts: Mapping[str, Tensor],
                 destination: Tensor) -> None:
    """The svdq.nvfp4 core row (`decode_schemes.py:464-489`)."""
    _check_destination(destination)
    _validate("svdq.nvfp4", params, parts, destination)
    ops = _ops(destination)
    rows, cols = (int(v) for v in destination.shape)
    weight = _part(torch, parts["weight"], destination).view(torch.uint8)
    scale = _part(torch, parts["scale"], destination).view(torch.uint8)
    second = _part(torch, parts["scale_2"], destination).reshape(-1).float()
    channel = parts.get("channel_scale")
    channel = None if channel is None else _part(torch, channel, destination)
    smooth = _part(torch, parts["pre_quant_scale"], destination)
    down = _part(torch, parts["lowrank_down"], destination)
    up = _part(torch, parts["lowrank_up"], destination)
    ops.decode_svdq(
        weight, scale, params["scale_layout"] == "cublas_128x4",
        params["nibble_order"] == "high_first", second, params["global_scale"] == "divide",
        channel, 0 if channel is None else _num(channel), smooth, _num(smooth), down, _num(down),
        up, _num(up), destination, rows, cols,
    )  # fmt: skip


@dataclass(frozen=True, slots=True)
class CoreDequant:
    """A core row's scheme -> float (`internal/encoding/adapters.py:33-102`): here `nvfp4` (with
    the optional per-column `pre_quant_scale`), `svdq.nvfp4` and `mxfp8`."""

    encoding: str = ""
    params: Params = ()

    @property
    def name(self) -> str:
        return f"cozy.{self.encoding}.cores/1"

    route = property(lambda self: "decoded_float")
    device_predicate = property(lambda self: "rocm.gfx950")
    schemes = property(lambda self: frozenset(CORE_ROWS))
    code_revision = property(lambda self: "1")
    suite = property(lambda self: "cores-decode")
    required = property(lambda self: CORE_ROWS[self.encoding].required)
    optional = property(lambda self: CORE_ROWS[self.encoding].optional)

    def supports(self, shape: Sequence[int], params: Mapping[str, object]) -> str:
        row = CORE_ROWS[self.encoding]
        unknown = sorted(set(params) - set(row.params))
        if unknown:
            return f"{row.scheme}: unknown params {unknown}"
        for key, values in row.params.items():
            if key not in params:
                return f"{row.scheme}: param {key} is missing"
            if not _allowed(values, params[key]):
                return f"{row.scheme}: param {key}={params[key]!r}"
        if len(shape) < 2:
            return f"{row.scheme} views rank 2 or more, not {tuple(shape)}"
        return ""

    def decode(self, torch: Any, parts: Mapping[str, Tensor], destination: Tensor) -> None:
        params = dict(self.params)
        if self.encoding == "mxfp8":
            _decode_mx(torch, params, parts, destination)
        elif self.encoding == "nvfp4":
            _decode_nvfp4(torch, params, parts, destination)
        else:
            _decode_svdq(torch, params, parts, destination)


def provider_for(scheme: str, params: Mapping[str, object] | Params = ()) -> Any:
    """The decode provider bound to `params` for `scheme`, or None: the formats providers for
    their schemes, the cores for nvfp4 (with AWQ smoothing) and svdq.nvfp4."""
    bound: Params = tuple(sorted(dict(params).items()))
    if scheme in ("fp8.tensorwise", "int8.tensorwise"):
        return TensorwiseDequant(scheme, bound)
    if scheme in ("fp8.rowwise", "int8.rowwise", "fp8.columnwise", "int8.columnwise"):
        return RowwiseDequant(scheme, bound)
    if scheme == "int8.convrot":
        return Int8ConvRotDequant(scheme, bound)
    if scheme in CORE_ROWS:
        return CoreDequant(scheme, bound)
    return None


def decode(torch: Any, scheme: str, params: Mapping[str, object], parts: Mapping[str, Tensor],
           destination: Tensor) -> None:
    """Decode a stored tensor into `destination`, refusing (ValueError) what `part_rule`
    refuses."""
    provider = provider_for(scheme, params)
    if provider is None:
        raise ValueError(f"no decode provider serves {scheme}")
    provider.decode(torch, parts, destination)

"""The stored-format decode providers (`cozyq.decode`, kernels in `csrc/decode.hip`).

CPU: the fill plane's part rules refuse every refusal case of the reference's vectors and accept
every decode case; the providers keep the reference's names, schemes, roles and messages.
GPU: every decode case of the reference's vectors bit-exact, then seeded shapes far larger than
the vectors (both kernel paths, every element code, scale dtype, grid, layout and destination)
bit-exact against the oracle's restatement of each law.
"""

from __future__ import annotations

import math

import pytest
import torch

import vectors
from cozyq import decode as dec
from oracle import laws

FILES = ("int8", "fp8", "mxfp8", "nvfp4", "svdq")
SCHEME = {"svdq": "svdq.nvfp4"}


def _scheme(case: dict) -> str:
    return case["encoding"]["scheme"]


def _all(kind: str) -> list[dict]:
    out = []
    for name in FILES:
        out += [c for c in vectors.cases(name) if (c["component"] == "refuse") == (kind == "refuse")]
    return out


# ----------------------------------------------------------------------------- CPU


@pytest.mark.parametrize("case", _all("refuse"), ids=lambda c: c["key"])
def test_part_rule_refuses_every_refusal_vector(case):
    why = dec.part_rule(_scheme(case), case["encoding"]["params"], case["shape"],
                        vectors.NAMES.get(case["dtype"], case["dtype"]), vectors.part_names(case))
    assert why, case["key"]


@pytest.mark.parametrize("case", _all("decode"), ids=lambda c: c["key"])
def test_part_rule_accepts_every_decode_vector(case):
    why = dec.part_rule(_scheme(case), case["encoding"]["params"], case["shape"],
                        vectors.NAMES[case["dtype"]], vectors.part_names(case))
    assert why == "", why


def test_provider_surface_matches_the_reference():
    """Names, suites, roles and code revisions of `internal/encoding/formats.py:438-868` and
    `internal/encoding/adapters.py:33-102`."""
    rows = {
        dec.TensorwiseDequant("fp8.tensorwise"): ("cozy.fp8-tensorwise.dequant/1", "fp8-tensorwise-decode"),
        dec.TensorwiseDequant("int8.tensorwise"): ("cozy.int8-tensorwise.dequant/1", "int8-tensorwise-decode"),
        dec.RowwiseDequant("fp8.rowwise"): ("cozy.fp8-rowwise.dequant/1", "fp8-rowwise-decode"),
        dec.RowwiseDequant("int8.rowwise"): ("cozy.int8.rowwise.dequant/1", "int8-rowwise-decode"),
        dec.columnwise(): ("cozy.fp8.columnwise.dequant/1", "fp8-columnwise-decode"),
        dec.MicroScaledDequant(): ("cozy.mxfp8.dequant/1", "mxfp8-decode"),
        dec.Int8ConvRotDequant(): ("cozy.int8-convrot.dequant/1", "int8-convrot-decode"),
        dec.Nvfp4Dequant(): ("cozy.nvfp4.dequant/1", "nvfp4-decode"),
        dec.CoreDequant("svdq.nvfp4"): ("cozy.svdq.nvfp4.cores/1", "cores-decode"),
    }  # fmt: skip
    for provider, (name, suite) in rows.items():
        assert (provider.name, provider.suite, provider.route) == (name, suite, "decoded_float")
    assert dec.columnwise().schemes == {"fp8.columnwise", "int8.columnwise"}
    assert dec.Nvfp4Dequant().required == {"weight", "scale", "scale_2"}
    assert dec.CoreDequant("svdq.nvfp4").optional == {"input_scale", "channel_scale"}


def test_supports_messages():
    conv = dec.Int8ConvRotDequant()
    params = {"rotation": "kron_regular_h4", "rotation_size": 256}
    assert conv.supports((4, 512), params) == ""
    assert "whole 256-column groups" in conv.supports((1, 64), params)
    assert "expected one of" in conv.supports((4, 512), {**params, "rotation_size": 32})
    assert "rank-2 weight" in dec.columnwise().supports((2, 4, 8), {})
    assert "two axes" in dec.RowwiseDequant().supports((8,), {})
    mx = {"block_size": 32, "scale_layout": "cublas_128x4"}
    assert "through the cores" in dec.MicroScaledDequant().supports((3, 80, 96), mx)
    nv = {"block_size": 16, "global_scale": "multiply", "nibble_order": "low_first",
          "scale_layout": "row_major"}  # fmt: skip
    assert "whole 16-column blocks" in dec.Nvfp4Dequant().supports((4, 40), nv)
    assert dec.CoreDequant("nvfp4").supports((4, 64), {**nv, "global_scale": "add"})


def test_decode_refuses_a_destination_off_the_gpu():
    parts = {"weight": torch.zeros(2, 32, dtype=torch.int8), "scale": torch.ones(2)}
    with pytest.raises(ValueError, match="on the GPU"):
        dec.RowwiseDequant("int8.rowwise").decode(torch, parts, torch.empty(2, 32))


def test_decode_refuses_what_the_part_rule_refuses():
    parts = {"weight": torch.zeros(2, 32, dtype=torch.int8), "scale": torch.ones(3)}
    with pytest.raises(ValueError, match="expected 2"):
        dec.decode(torch, "int8.rowwise", {}, parts, torch.empty(2, 32))


# ----------------------------------------------------------------------------- GPU

CUDA = "cuda:0"


def _to(parts: dict[str, torch.Tensor]) -> dict[str, torch.Tensor]:
    return {r: t.to(CUDA) for r, t in parts.items()}


def _gpu_decode(scheme: str, params: dict, parts: dict, shape, dtype) -> torch.Tensor:
    out = torch.empty(shape, dtype=dtype, device=CUDA)
    dec.decode(torch, scheme, params, _to(parts), out)
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.gpu
@pytest.mark.parametrize("case", _all("decode"), ids=lambda c: c["key"])
def test_gpu_decode_vectors_bit_exact(case):
    """Every decode case the reference's vectors hold, through the provider, on the GPU."""
    got = _gpu_decode(_scheme(case), case["encoding"]["params"], vectors.parts(case),
                      case["shape"], vectors.DTYPES[case["dtype"]])  # fmt: skip
    assert vectors.same(got, case), case["key"]


def _bits_equal(got: torch.Tensor, want: torch.Tensor) -> None:
    assert got.shape == want.shape and got.dtype == want.dtype
    nan = torch.isnan(got.float())
    assert torch.equal(nan, torch.isnan(want.float()))
    bits = torch.int32 if got.element_size() == 4 else torch.int16
    diff = (got[~nan].contiguous().view(bits) != want[~nan].contiguous().view(bits)).sum()
    assert int(diff) == 0, f"{int(diff)} of {got.numel()} elements differ"


OUTS = (torch.float32, torch.bfloat16, torch.float16)
SCALES = (torch.float32, torch.bfloat16, torch.float16)


def _codes(kind: str, shape, g: torch.Generator) -> torch.Tensor:
    raw = torch.randint(0, 256, shape, generator=g, dtype=torch.int32).to(torch.uint8)
    if kind == "i8":
        return raw.view(torch.int8)
    if kind == "e4m3":
        return raw.view(torch.float8_e4m3fn)  # every code, NaN included
    return raw.view(torch.float8_e5m2)


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["i8", "e4m3", "e5m2"])
@pytest.mark.parametrize("shape", [(1024, 4096), (96, 1000), (7, 3, 48)])
def test_gpu_row_column_tensor_decode_against_the_oracle(kind, shape):
    """Rows of whole 16-element runs take the vector path; 1000-column rows the element path."""
    g = torch.Generator().manual_seed(10 * ("i8", "e4m3", "e5m2").index(kind) + len(shape))
    rows, cols = math.prod(shape[:-1]), shape[-1]
    weight = _codes(kind, shape, g)
    scheme = "int8" if kind == "i8" else "fp8"
    for i, dtype in enumerate(OUTS):
        sdt = SCALES[(i + 1) % 3]
        row_scale = (torch.rand(rows, generator=g) * 0.02 + 1e-4).to(sdt)
        got = _gpu_decode(f"{scheme}.rowwise", {}, {"weight": weight, "scale": row_scale}, shape,
                          dtype)  # fmt: skip
        _bits_equal(got, laws.decode_rowwise(weight.reshape(rows, cols), row_scale, dtype).reshape(shape))
        one = torch.tensor(0.0123, dtype=sdt)
        got = _gpu_decode(f"{scheme}.tensorwise", {}, {"weight": weight, "scale": one}, shape, dtype)
        _bits_equal(got, laws.decode_tensorwise(weight, one, dtype))
        if len(shape) == 2:
            col_scale = (torch.rand(cols, generator=g) + 0.5).to(sdt)
            got = _gpu_decode(f"{scheme}.columnwise", {}, {"weight": weight, "scale": col_scale},
                              shape, dtype)  # fmt: skip
            _bits_equal(got, laws.decode_columnwise(weight, col_scale, dtype))


def _e8m0(shape, g) -> torch.Tensor:
    b = torch.randint(100, 140, shape, generator=g, dtype=torch.int32)
    b[..., 0] = 0  # 2^-127, the subnormal
    return b.to(torch.uint8)


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["row_major", "cublas_128x4"])
@pytest.mark.parametrize("shape", [(3072, 3072), (300, 1000), (3, 200, 96)])
@pytest.mark.parametrize("kind", ["e4m3", "e5m2"])
def test_gpu_mx_decode_against_the_oracle(layout, shape, kind):
    g = torch.Generator().manual_seed(11)
    stack = math.prod(shape[:-2]) if len(shape) > 2 else 1
    rows, cols = shape[-2], shape[-1]
    blocks = -(-cols // 32)
    weight = _codes(kind, shape, g)
    grids = [_e8m0((rows, blocks), g) for _ in range(stack)]
    if layout == "cublas_128x4":
        scale = torch.stack([laws.to_blocked(gr).reshape(laws._blocked_shape(rows, blocks))
                             for gr in grids]).reshape(*shape[:-2], *laws._blocked_shape(rows, blocks))  # fmt: skip
    else:
        scale = torch.stack(grids).reshape(*shape[:-1], blocks)
    params = {"block_size": 32, "scale_layout": layout}
    for dtype in OUTS:
        got = _gpu_decode("mxfp8", params, {"weight": weight, "scale": scale}, shape, dtype)
        want = torch.stack([laws.decode_mxfp8(weight.reshape(stack, rows, cols)[e], grids[e],
                                              "row_major", dtype) for e in range(stack)])  # fmt: skip
        _bits_equal(got, want.reshape(shape))


@pytest.mark.gpu
@pytest.mark.parametrize("size", laws.ROTATION_SIZES)
def test_gpu_convrot_decode_every_rotation_size(size):
    """4 … 65536: in registers, across lanes (DPP, ds_bpermute) and across waves (LDS)."""
    g = torch.Generator().manual_seed(size)
    cols = max(size, 4096) if size <= 4096 else size
    rows = max(2, (1 << 21) // cols)
    weight = torch.randint(-127, 128, (rows, cols), generator=g, dtype=torch.int8)
    weight[0, :] = 127  # the largest sums
    weight[1, :] = -127
    params = {"rotation": "kron_regular_h4", "rotation_size": size}
    for i, dtype in enumerate(OUTS):
        scale = (torch.rand(rows, generator=g) * 1e-3).to(SCALES[i])
        got = _gpu_decode("int8.convrot", params, {"weight": weight, "scale": scale},
                          (rows, cols), dtype)  # fmt: skip
        _bits_equal(got, laws.decode_int8_convrot(weight, scale, size, dtype))


@pytest.mark.gpu
@pytest.mark.parametrize("size", [4, 16, 256])
def test_gpu_convrot_decode_ragged_and_unaligned(size):
    """Row counts whose total is not a multiple of 64, and a destination at an odd offset."""
    g = torch.Generator().manual_seed(5)
    rows, cols = 7, size * 3
    weight = torch.randint(-127, 128, (rows, cols), generator=g, dtype=torch.int8)
    scale = torch.rand(rows, generator=g)
    params = {"rotation": "kron_regular_h4", "rotation_size": size}
    want = laws.decode_int8_convrot(weight, scale, size, torch.bfloat16)
    slab = torch.empty(rows * cols + 1, dtype=torch.bfloat16, device=CUDA)
    out = slab[1:].view(rows, cols)
    dec.decode(torch, "int8.convrot", params, _to({"weight": weight, "scale": scale}), out)
    torch.cuda.synchronize()
    _bits_equal(out.cpu(), want)


def _nvfp4_parts(rows: int, cols: int, g: torch.Generator, tiled: bool, stack: int = 1):
    weight = torch.randint(0, 256, (stack, rows, cols // 2), generator=g, dtype=torch.int32)
    weight = weight.to(torch.uint8)
    grids = [(torch.rand(rows, cols // 16, generator=g) * 4 + 0.01).to(torch.float8_e4m3fn)
             for _ in range(stack)]  # fmt: skip
    if tiled:
        shape = laws._blocked_shape(rows, cols // 16)
        scale = torch.stack([laws.to_blocked(gr.view(torch.uint8)).view(torch.float8_e4m3fn)
                             .reshape(shape) for gr in grids])  # fmt: skip
    else:
        scale = torch.stack(grids)
    return weight, scale, grids


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["row_major", "cublas_128x4"])
@pytest.mark.parametrize("order", ["low_first", "high_first"])
@pytest.mark.parametrize("mode", ["multiply", "divide"])
def test_gpu_nvfp4_decode_against_the_oracle(layout, order, mode):
    g = torch.Generator().manual_seed(7)
    rows, cols, stack = 1000, 2048, 3
    weight, scale, grids = _nvfp4_parts(rows, cols, g, layout == "cublas_128x4", stack)
    second = torch.rand(stack, generator=g) + 0.25
    post = (torch.rand(cols, generator=g) + 0.5).to(torch.bfloat16)
    params = {"block_size": 16, "global_scale": mode, "nibble_order": order, "scale_layout": layout}
    parts = {"weight": weight, "scale": scale, "scale_2": second, "pre_quant_scale": post}
    for dtype in OUTS:
        got = _gpu_decode("nvfp4", params, parts, (stack, rows, cols), dtype)
        want = torch.stack([laws.decode_nvfp4(weight[e], grids[e], second[e], "row_major",
                                              order == "high_first", mode == "divide", post,
                                              dtype) for e in range(stack)])  # fmt: skip
        _bits_equal(got, want)


@pytest.mark.gpu
@pytest.mark.parametrize("rank", [1, 32, 128])
@pytest.mark.parametrize("layout", ["row_major", "cublas_128x4"])
def test_gpu_svdq_decode_against_the_oracle(rank, layout):
    g = torch.Generator().manual_seed(rank)
    rows, cols = 768, 1024
    weight, scale, grids = _nvfp4_parts(rows, cols, g, layout == "cublas_128x4")
    second = torch.tensor(0.37)
    channel = (torch.rand(rows, generator=g) * 2).to(torch.float8_e4m3fn)
    smooth = torch.rand(cols, generator=g) + 0.5
    down = (torch.randn(rank, cols, generator=g) * 0.05).to(torch.bfloat16)
    up = (torch.randn(rows, rank, generator=g) * 0.05).to(torch.float16)
    params = {"block_size": 16, "global_scale": "multiply", "nibble_order": "low_first",
              "scale_layout": layout}  # fmt: skip
    parts = {"weight": weight[0], "scale": scale[0], "scale_2": second, "channel_scale": channel,
             "pre_quant_scale": smooth, "lowrank_down": down, "lowrank_up": up}  # fmt: skip
    for dtype in OUTS:
        got = _gpu_decode("svdq.nvfp4", params, parts, (rows, cols), dtype)
        want = laws.decode_svdq_nvfp4(weight[0], grids[0], second, "row_major", False, False,
                                      channel, smooth, down, up, dtype)  # fmt: skip
        _bits_equal(got, want)

"""Pins the CPU oracle (`oracle/laws.py`) to things other than itself: the reference's own decode
vectors (`tests/golden/ref_*_vectors.json`, copied from cozy-runtime's
`internal/encoding/vectors/cases/`), closed forms, brute force over every bf16/fp16 input, and an
independent bit-level E4M3 encoder."""

from __future__ import annotations

import base64
import json
import math
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest
import torch

import vectors
from oracle import laws

GOLDEN = Path(__file__).resolve().parent / "golden"
DTYPES = {"F32": torch.float32, "BF16": torch.bfloat16, "F16": torch.float16, "I8": torch.int8,
          "F8_E4M3": torch.float8_e4m3fn, "F8_E5M2": torch.float8_e5m2, "F8_E8M0": torch.uint8}


def _tensor(bits: str, dtype: str, shape: list[int]) -> torch.Tensor:
    raw = bytearray(base64.b64decode(bits))
    return torch.frombuffer(raw, dtype=DTYPES[dtype]).reshape(shape) if raw else \
        torch.empty(shape, dtype=DTYPES[dtype])


def _cases(name: str, component: str) -> list[dict]:
    data = json.loads((GOLDEN / f"ref_{name}_vectors.json").read_text())
    return [c for c in data["cases"] if c["component"] == component]


def _parts(case: dict) -> dict[str, torch.Tensor]:
    return {p["role"]: _tensor(p["bits"], p["dtype"], p["shape"]) for p in case["parts"]}


def _expect_bytes(case: dict) -> bytes:
    return base64.b64decode(case["expect"])


def _same(got: torch.Tensor, case: dict) -> bool:
    """Bit-for-bit equality with the vector's expected output, except that a NaN matches any
    NaN (NaN payload bits are not part of any law here)."""
    want = torch.frombuffer(bytearray(_expect_bytes(case)), dtype=got.dtype).reshape(got.shape)
    nan = torch.isnan(got.float())
    if not torch.equal(nan, torch.isnan(want.float())):
        return False
    bits = torch.int32 if got.element_size() == 4 else torch.int16
    return torch.equal(got[~nan].contiguous().view(bits), want[~nan].contiguous().view(bits))


# ----------------------------------------------------------------- reference vectors


@pytest.mark.parametrize("case", _cases("int8", "int8.convrot"), ids=lambda c: c["key"])
def test_int8_convrot_decode_vectors(case):
    """The reference's int8.convrot decode vectors pin the rotation's signs and index order."""
    parts = _parts(case)
    size = case["encoding"]["params"]["rotation_size"]
    rows, cols = case["shape"]
    got = laws.decode_int8_convrot(parts["weight"].reshape(rows, cols), parts["scale"], size,
                                   DTYPES[case["dtype"]])  # fmt: skip
    assert _same(got, case)


@pytest.mark.parametrize("case", _cases("int8", "int8.rowwise"), ids=lambda c: c["key"])
def test_int8_rowwise_decode_vectors(case):
    parts = _parts(case)
    got = laws.decode_rowwise(parts["weight"], parts["scale"], DTYPES[case["dtype"]])
    assert _same(got, case)


@pytest.mark.parametrize("case", _cases("fp8", "fp8.rowwise"), ids=lambda c: c["key"])
def test_fp8_rowwise_decode_vectors(case):
    """Pins the E4M3 and E5M2 element values and the float32-then-one-cast rounding."""
    parts = _parts(case)
    shape = case["shape"]
    rows = int(np.prod(shape[:-1]))
    got = laws.decode_rowwise(parts["weight"].reshape(rows, shape[-1]), parts["scale"].reshape(-1),
                              DTYPES[case["dtype"]])  # fmt: skip
    assert _same(got, case)


@pytest.mark.parametrize("case", _cases("mxfp8", "mxfp8"), ids=lambda c: c["key"])
def test_mxfp8_decode_vectors(case):
    """Pins the E8M0 multipliers, ragged last blocks and the cuBLAS 128x4 layout."""
    parts = _parts(case)
    shape = case["shape"]
    layout = case["encoding"]["params"]["scale_layout"]
    dtype = DTYPES[case["dtype"]]
    weight, scale = parts["weight"], parts["scale"]
    if len(shape) == 3:  # an expert stack decodes one matrix at a time
        got = torch.stack([laws.decode_mxfp8(weight[e], scale[e], layout, dtype)
                           for e in range(shape[0])])  # fmt: skip
    else:
        got = laws.decode_mxfp8(weight, scale, layout, dtype)
    assert _same(got, case)


@pytest.mark.parametrize(
    "case", vectors.cases("fp8", "fp8.tensorwise") + vectors.cases("int8", "int8.tensorwise"),
    ids=lambda c: c["key"])
def test_tensorwise_decode_vectors(case):
    parts = vectors.parts(case)
    got = laws.decode_tensorwise(parts["weight"], parts["scale"], DTYPES[case["dtype"]])
    assert vectors.same(got, case)


@pytest.mark.parametrize(
    "case", vectors.cases("fp8", "fp8.columnwise") + vectors.cases("int8", "int8.columnwise"),
    ids=lambda c: c["key"])
def test_columnwise_decode_vectors(case):
    parts = vectors.parts(case)
    got = laws.decode_columnwise(parts["weight"], parts["scale"], DTYPES[case["dtype"]])
    assert vectors.same(got, case)


def _nvfp4_oracle(case: dict) -> torch.Tensor:
    """The nvfp4 law over a case's parts: one matrix at a time for a stack (each with its own
    scale_2 and, under cuBLAS tiles, its own grid)."""
    parts, params = vectors.parts(case), case["encoding"]["params"]
    shape = case["shape"]
    rows, cols = shape[-2], shape[-1]
    stack = int(np.prod(shape[:-2])) if len(shape) > 2 else 1
    weight = parts["weight"].reshape(stack, rows, cols // 2)
    scale = parts["scale"].reshape(stack, -1)
    second = parts["scale_2"].reshape(-1)
    out = [laws.decode_nvfp4(weight[e], scale[e], second[e if second.numel() > 1 else 0],
                             params["scale_layout"], params["nibble_order"] == "high_first",
                             params["global_scale"] == "divide", parts.get("pre_quant_scale"),
                             DTYPES[case["dtype"]]) for e in range(stack)]  # fmt: skip
    return torch.stack(out).reshape(shape)


@pytest.mark.parametrize("case", vectors.cases("nvfp4", "nvfp4"), ids=lambda c: c["key"])
def test_nvfp4_decode_vectors(case):
    """Pins E2M1's values, both nibble orders, multiply/divide second-level scales, the E4M3
    block scales in both layouts, per-matrix scale_2 and AWQ's per-column pre_quant_scale."""
    assert vectors.same(_nvfp4_oracle(case), case)


@pytest.mark.parametrize("case", vectors.cases("svdq", "svdq"), ids=lambda c: c["key"])
def test_svdq_nvfp4_decode_vectors(case):
    """Pins the svdq.nvfp4 decode: channel scale (f32 or E4M3), smoothing, and the low-rank
    term added product by product in rank order."""
    parts, params = vectors.parts(case), case["encoding"]["params"]
    got = laws.decode_svdq_nvfp4(
        parts["weight"], parts["scale"], parts["scale_2"], params["scale_layout"],
        params["nibble_order"] == "high_first", params["global_scale"] == "divide",
        parts.get("channel_scale"), parts["pre_quant_scale"], parts["lowrank_down"],
        parts["lowrank_up"], DTYPES[case["dtype"]])  # fmt: skip
    assert vectors.same(got, case)


def test_svdq_decode_rank_order_is_pinned():
    """A plausible slip — one fused sum of the low-rank products instead of adding each rounded
    product in turn — changes the result on values chosen to expose it, so the vectors above
    hold the order, not just the sum."""
    torch.manual_seed(3)
    rows, cols, rank = 4, 16, 8
    weight = torch.zeros(rows, cols // 2, dtype=torch.uint8)
    scale = torch.ones(rows, 1).to(torch.float8_e4m3fn)
    up = torch.randn(rows, rank) * 1e3
    down = torch.randn(rank, cols) * 1e-3
    smooth = torch.ones(cols)
    law = laws.decode_svdq_nvfp4(weight, scale, torch.tensor(1.0), "row_major", False, False,
                                 None, smooth, down, up, torch.float32)  # fmt: skip
    fused = (up.double() @ down.double()).float()
    assert not torch.equal(law, fused)


def test_blocked_layout_round_trip():
    grid = torch.randint(0, 255, (300, 7), dtype=torch.uint8)
    blocked = laws.to_blocked(grid)
    assert blocked.numel() == 384 * 8
    assert torch.equal(laws.from_blocked(blocked, 300, 7), grid)


# -------------------------------------------------------------------- closed forms


def _kron_h(size: int) -> np.ndarray:
    h4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.int64)
    h2 = np.array([[1, 1], [1, -1]], dtype=np.int64)
    factors = [h2, h4, h4, h4] if size == 128 else [h4] * int(round(math.log(size, 4)))
    out = np.ones((1, 1), dtype=np.int64)
    for f in factors:
        out = np.kron(out, f)
    return out


@pytest.mark.parametrize("size", [4, 16, 64, 256, 1024, 128])
def test_hadamard_is_the_kronecker_matrix(size):
    """The staged rotation equals x·H for H the Kronecker product, outer factor first; H is
    symmetric and H·H = n·I."""
    h = _kron_h(size)
    assert np.array_equal(h, h.T)
    assert np.array_equal(h @ h, size * np.eye(size, dtype=np.int64))
    x = torch.randint(-1000, 1000, (3, 2 * size), dtype=torch.int64)
    got = laws.hadamard(x, size).numpy()
    want = np.concatenate([x[:, :size].numpy() @ h, x[:, size:].numpy() @ h], axis=1)
    assert np.array_equal(got, want)


def test_hadamard_float_stage_order_is_associated_left_to_right():
    """The float32 rotation differs from other evaluation orders on some inputs and equals the
    stated one: ((a+b)+c)-d per output, outer stage first (formats.py:667-671). A plausible
    mistake, (a+b)+(c-d), changes bits here."""
    gen = torch.Generator().manual_seed(7)
    x = (torch.randn(64, 256, generator=gen) * torch.logspace(-4, 4, 256)).float()
    ref = laws.hadamard(x, 256)
    work = x.reshape(-1, 4, 4, 4, 4)
    for axis in range(1, 5):
        a, b, c, d = work.unbind(axis)
        work = torch.stack(((a + b) + (c - d), (a + b) - (c - d), (a - b) + (c + d),
                            (b + c) + (d - a)), axis)  # fmt: skip
    other = work.reshape(x.shape)
    assert not torch.equal(ref, other)
    exact = laws.hadamard(x.double(), 256)
    assert torch.allclose(ref.double(), exact, rtol=0, atol=1e-3 * exact.abs().max().item())


def test_int32_gemm_matches_numpy_int64():
    gen = torch.Generator().manual_seed(1)
    q = torch.randint(-127, 128, (37, 512), generator=gen, dtype=torch.int8)
    w = torch.randint(-127, 128, (24, 512), generator=gen, dtype=torch.int8)
    got = laws.int32_gemm(q, w)
    want = q.numpy().astype(np.int64) @ w.numpy().astype(np.int64).T
    assert np.array_equal(got.numpy().astype(np.int64), want)


# Exact rational arithmetic with an independent round-to-nearest-even onto a binary grid: the
# int8 epilogue's rounding sequence is checked against it, not against torch.
_FORMATS = {torch.float32: (24, -126), torch.bfloat16: (8, -126), torch.float16: (11, -14)}


def _rne(v: Fraction, dtype: torch.dtype) -> Fraction:
    """`v` rounded to nearest (ties to even) in `dtype` (significand bits, least normal
    exponent; subnormals kept; the cases here stay far from overflow)."""
    if v == 0:
        return Fraction(0)
    bits, emin = _FORMATS[dtype]
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp = Fraction(2) ** (max(e, emin) - bits + 1)
    units = a / ulp
    whole = units.numerator // units.denominator
    rest = units - whole
    if rest > Fraction(1, 2) or (rest == Fraction(1, 2) and whole % 2 == 1):
        whole += 1
    return (whole * ulp) if v > 0 else -(whole * ulp)


def _frac(t: torch.Tensor) -> list[Fraction]:
    return [Fraction(v) for v in t.double().reshape(-1).tolist()]


def _epilogue_cases(dtype: torch.dtype):
    """int32 accumulators (a third of them past 2**24, where `acc.float()` rounds), row and
    column scales that are not powers of two, and biases of the output dtype."""
    gen = torch.Generator().manual_seed(20261202)
    rows, cols = 48, 64
    acc = torch.randint(-(1 << 20), 1 << 20, (rows, cols), generator=gen, dtype=torch.int64)
    big = torch.randint(1 << 24, 49_000_000, (rows, cols), generator=gen, dtype=torch.int64)
    acc = torch.where(torch.rand(rows, cols, generator=gen) < 0.33, big * acc.sign(), acc)
    acc = acc.to(torch.int32)
    xs = ((torch.rand(rows, 1, generator=gen) + 0.3) * 1e-2).float()
    ws = ((torch.rand(cols, generator=gen) + 0.3) * 1e-3).float()
    bias = (torch.randn(cols, generator=gen) * 4).to(dtype)
    return acc, xs, ws, bias


def test_int8_epilogue_rounding_sequence():
    """`laws.int8_epilogue` against the reference's sequence evaluated in exact rationals
    (`internal/int8_linear.py:447-448` + `:276`): rne32(acc), rne32(· xs), rne32(· ws), one
    rounding to the output dtype, then the bias added in that dtype (a float32 sum rounded
    once more). A float32 output shows the products' order bit for bit; bf16 and fp16 outputs
    show the cast and the bias step. Each plausible variant — xs·ws first, ws first, no
    rounding of the accumulator, one fused multiply-add with the bias, the bias added before the
    cast — changes some of these bits, so this pins the order and not only the values."""
    f32 = torch.float32
    differs: dict[str, int] = {}
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        acc, xs, ws, bias = _epilogue_cases(dtype)
        got = laws.int8_epilogue(acc, xs, ws, bias, dtype)
        a_, x_, w_, b_ = _frac(acc), _frac(xs), _frac(ws), _frac(bias)
        cols = acc.shape[1]

        def out(p, b):  # the cast, then the bias in the output dtype
            return _rne(_rne(_rne(p, dtype) + b, f32), dtype)

        def law(a, x, w, b):
            return out(_rne(_rne(_rne(a, f32) * x, f32) * w, f32), b)

        variants = {
            "xs*ws first": lambda a, x, w, b: out(_rne(_rne(a, f32) * _rne(x * w, f32), f32), b),
            "ws first": lambda a, x, w, b: out(_rne(_rne(_rne(a, f32) * w, f32) * x, f32), b),
            "exact accumulator": lambda a, x, w, b: out(_rne(_rne(a * x, f32) * w, f32), b),
            "fma with bias": lambda a, x, w, b: _rne(_rne(_rne(_rne(a, f32) * x, f32) * w + b, f32), dtype),
            "bias before cast": lambda a, x, w, b: _rne(_rne(_rne(_rne(_rne(a, f32) * x, f32) * w, f32) + b, f32), dtype),
        }
        want = []
        for i, a in enumerate(a_):
            r, c = divmod(i, cols)
            args = (a, x_[r], w_[c], b_[c])
            expect = law(*args)
            want.append(expect)
            for name, fn in variants.items():
                differs[name] = differs.get(name, 0) + (fn(*args) != expect)
        assert _frac(got) == want, dtype
    assert all(n > 0 for n in differs.values()), differs


def test_int8_linear_uses_the_pinned_epilogue():
    """`int8_linear` is quantize → exact int32 product → the epilogue pinned above."""
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(5, 512, generator=gen).to(torch.bfloat16)
    data = torch.randint(-127, 128, (24, 512), generator=gen, dtype=torch.int8)
    scale = (torch.rand(24, generator=gen) + 0.5) * 1e-3
    bias = torch.randn(24, generator=gen).to(torch.bfloat16)
    q, s = laws.quantize_rows_int8(x, 256)
    want = laws.int8_epilogue(laws.int32_gemm(q, data), s, scale, bias, torch.bfloat16)
    assert torch.equal(laws.int8_linear(x, data, scale, bias, torch.bfloat16), want)


def test_gelu_tanh_against_library_routine():
    """`laws.gelu_tanh` (float32) against torch's tanh-approximate GELU evaluated in float64, on
    every bf16 value in [-12, 12]: within 4 float32 ulps of the result, plus |y|·2**-23 for the
    cancellation in 1 + tanh(u) as the reference writes it (`internal/prebuilt.py:775`: f32
    tanh(u) near −1 carries 2**-25 of absolute error), plus 2**-126 (the reference's constant
    0.79788456 and √(2/π) agree to 1e-9 relative); exactly 0 at 0, and the odd-part identity
    gelu(y) − gelu(−y) = y. A wrong constant, a dropped ½ or the erf form miss these bounds."""
    raw = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float()
    y = raw[torch.isfinite(raw) & (raw.abs() <= 12)]
    got = laws.gelu_tanh(y).double()
    want = torch.nn.functional.gelu(y.double(), approximate="tanh")
    eps = torch.finfo(torch.float32).eps
    bound = 4 * eps * want.abs() + y.double().abs() * 2.0**-23 + 2.0**-126
    assert ((got - want).abs() <= bound).all()
    wrong = 0.5 * y.double() * (1 + torch.tanh(0.79788456 * (y.double() + 0.0447 * y.double() ** 3)))
    assert ((wrong - want).abs() > bound).any()
    erf = torch.nn.functional.gelu(y.double())
    assert ((erf - want).abs() > bound).sum() > 1000
    assert laws.gelu_tanh(torch.zeros(1)).item() == 0.0
    pos = y[y > 0]
    odd = (laws.gelu_tanh(pos).double() - laws.gelu_tanh(-pos).double() - pos.double()).abs()
    assert (odd <= 4 * torch.finfo(torch.float32).eps * pos.double()).all()


@pytest.mark.parametrize("rotation", [0, 128, 256])
def test_int8_quantize_round_trip(rotation):
    """Codes reach ±127 at each row's maximum, every element dequantizes within half a step of
    the rotated (normalized) row, and all-zero rows give zero codes."""
    gen = torch.Generator().manual_seed(2)
    x = torch.randn(9, 1024, generator=gen).to(torch.bfloat16)
    x[3] = 0
    q, s = laws.quantize_rows_int8(x, rotation)
    assert q.dtype == torch.int8 and s.shape == (9, 1)
    xf = x.float().double()
    if rotation:
        rotated = laws.hadamard(xf, rotation) / math.sqrt(rotation)
    else:
        rotated = xf
    err = (q.double() * s.double() - rotated).abs()
    assert (err <= s.double() * 0.5 * (1 + 1e-5) + 1e-30).all()
    live = [r for r in range(9) if r != 3]
    assert (q[live].abs().amax(-1) == 127).all()
    assert (q[3] == 0).all()


# --------------------------------------------------------------------- E4M3 / E8M0


def _all_half_values(dtype: torch.dtype) -> torch.Tensor:
    raw = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(dtype)
    return raw[torch.isfinite(raw.float())].float()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_e4m3_cast_matches_bit_encoder_on_every_input(dtype):
    """torch's cast (the law's) and the independent integer encoder agree on every bf16/fp16
    value in [-448, 448]."""
    v = _all_half_values(dtype)
    v = v[v.abs() <= 448]
    got = v.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    want = laws.e4m3_bits_numpy(v.numpy())
    assert np.array_equal(got, want)


def _e4m3_midpoints() -> np.ndarray:
    codes = np.arange(0, 0x7F, dtype=np.uint8)
    vals = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    mids = (vals[:-1] + vals[1:]) / 2
    f32 = mids.astype(np.float32)
    bits = f32.view(np.uint32)
    near = np.concatenate([f32, (bits + 1).view(np.float32), (bits - 1).view(np.float32)])
    near = np.concatenate([near, -near, vals.astype(np.float32), -vals.astype(np.float32)])
    return near[np.abs(near) <= 448]


def test_e4m3_cast_at_round_to_nearest_even_midpoints():
    v = _e4m3_midpoints()
    got = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, laws.e4m3_bits_numpy(v))


def _exact_mx_byte(amax: np.ndarray) -> np.ndarray:
    """clamp(ceil(log2(amax/448)) + 127, 0, 254) with the ceiling taken exactly."""
    q = (amax.astype(np.float32) / np.float32(448.0)).astype(np.float64)
    mant, exp = np.frexp(q)  # q = mant·2^exp, mant in [0.5, 1)
    e = np.where(mant == 0.5, exp - 1, exp)
    b = np.clip(e + 127, 0, 254)
    return np.where(amax > 0, b, 0).astype(np.uint8)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_mx_exponent_every_block_max(dtype):
    """`mx_quantize`'s byte (torch log2 + ceil, the law) equals the exact integer ceiling for
    every positive bf16/fp16 block maximum."""
    v = _all_half_values(dtype)
    v = v[v > 0]
    block = torch.zeros(v.numel(), 32)
    block[:, 5] = v
    _, byte = laws.mx_quantize(block.to(dtype))
    assert np.array_equal(byte.reshape(-1).numpy(), _exact_mx_byte(v.numpy()))


def test_mx_round_trip_and_zero_blocks():
    gen = torch.Generator().manual_seed(3)
    x = (torch.randn(8, 256, generator=gen) * torch.logspace(-6, 6, 8).reshape(-1, 1)).to(torch.bfloat16)
    x[2, 32:64] = 0
    p, b = laws.mx_quantize(x)
    assert b[2, 1] == 0 and (p[2, 32:64].float() == 0).all()
    got = laws.mx_dequantize(p, b)
    blocks = x.float().reshape(8, 8, 32)
    mult = laws.e8m0_multipliers(b).unsqueeze(-1)
    # scaled block maxima land in (224, 448]; half an e4m3 ulp there is at most 16
    top = (blocks.abs().amax(-1, keepdim=True) / mult)
    assert ((top > 224) | (top == 0)).all() and (top <= 448).all()
    err = (got.reshape(8, 8, 32) - blocks).abs()
    assert (err <= 16 * mult).all()
    assert p.float().abs().max() <= 448


def test_e8m0_multipliers_by_construction():
    byte = torch.arange(0, 256, dtype=torch.int32).to(torch.uint8)
    got = laws.e8m0_multipliers(byte)
    assert got[0].item() == 2.0 ** -127
    assert all(got[b].item() == 2.0 ** (b - 127) for b in range(1, 255))
    assert math.isnan(got[255].item())


# ------------------------------------------------------------------ int4-g64 (build law)


def test_int4_quantize_round_trip_and_edges():
    gen = torch.Generator().manual_seed(4)
    v = torch.randn(6, 256, generator=gen) * torch.logspace(-3, 3, 6).reshape(-1, 1)
    v[1, 64:128] = 0
    q, s = laws.int4_quantize(v)
    assert q.dtype == torch.int8 and s.dtype == torch.float16 and s.shape == (6, 4)
    assert int(q.min()) >= -8 and int(q.max()) <= 7
    assert (q[1, 64:128] == 0).all() and s[1, 1] == 0
    deq = (q.float().reshape(6, 4, 64) * s.float().unsqueeze(-1)).reshape(6, 256)
    assert ((deq - v).abs() <= s.float().repeat_interleave(64, 1) * 0.5 + 1e-30).all()


def test_int4_quantize_brute_force_small():
    """Every code is the nearest of −8..7 steps to v/s (ties to even), s = fp16(amax/7)."""
    gen = torch.Generator().manual_seed(5)
    v = torch.randn(4, 64, generator=gen)
    q, s = laws.int4_quantize(v)
    for r in range(4):
        scale = float(s[r, 0])
        assert scale == float(np.float16(np.float32(v[r].abs().max()) / np.float32(7.0)))
        for k in range(64):
            t = float(np.float32(v[r, k]) / np.float32(scale))
            best = min(range(-8, 8), key=lambda c: (abs(c - t), c % 2))
            assert int(q[r, k]) == best


def test_int4_pack_round_trip():
    q = torch.randint(-8, 8, (5, 128), dtype=torch.int8)
    packed = laws.pack_int4(q)
    assert packed.shape == (5, 64)
    assert int(packed[0, 0]) & 0xF == int(q[0, 0]) & 0xF
    assert torch.equal(laws.unpack_int4(packed), q)


# --------------------------------------------------------------- SVDQuant W4A4 structure


def test_svdq_smooth_closed_forms():
    """Unit smoothing returns x itself; a power-of-two p scales exactly; a general p lands every
    value on the bf16 grid (the rounding is taken) within half a bf16 step of the product."""
    gen = torch.Generator().manual_seed(6)
    x = torch.randn(3, 128, generator=gen).to(torch.bfloat16)
    assert torch.equal(laws.svdq_smooth(x, torch.ones(128)), x.float())
    assert torch.equal(laws.svdq_smooth(x, torch.full((128,), 0.25)), x.float() * 0.25)
    p = torch.rand(128, generator=gen) * 1.5 + 0.5
    got = laws.svdq_smooth(x, p)
    assert (got.view(torch.int32) & 0xFFFF).eq(0).all()
    exact = x.double() * p.double()
    assert ((got.double() - exact).abs() <= exact.abs() * 2.0 ** -8).all()
    assert not torch.equal(got, (x.float() * p))  # the bf16 rounding is taken


def test_svdq_down_one_hot_and_integer():
    """A one-hot down row picks one input column; integer-valued operands sum exactly (numpy
    int64); an fp16 x casts down to fp16 first, so a bf16 value below fp16's range vanishes."""
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(5, 192, generator=gen).to(torch.bfloat16)
    down = torch.zeros(16, 192, dtype=torch.bfloat16)
    cols = torch.randperm(192, generator=gen)[:16]
    down[torch.arange(16), cols] = 1
    assert torch.equal(laws.svdq_down(x, down), x[:, cols])
    xi = torch.randint(-20, 21, (6, 256), generator=gen)
    di = torch.randint(-20, 21, (32, 256), generator=gen)
    want = xi.numpy().astype(np.int64) @ di.numpy().astype(np.int64).T
    got = laws.svdq_down(xi.to(torch.bfloat16), di.to(torch.bfloat16))
    assert torch.equal(got, torch.from_numpy(want).to(torch.bfloat16))
    xh = torch.ones(1, 64, dtype=torch.float16)
    tiny = torch.full((16, 64), 1e-9, dtype=torch.bfloat16)  # below fp16's least subnormal / 2
    assert laws.svdq_down(xh, tiny).eq(0).all()
    assert laws.svdq_down(xh.to(torch.bfloat16), tiny).ne(0).all()


def _on_grid(gen: torch.Generator, rows: int, cols: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Values exactly on the int4 grid: per 64-group codes with ±7 present and a power-of-two
    step, so that int4_quantize gives back these codes and step."""
    q = torch.randint(-7, 8, (rows, cols), generator=gen)
    q[:, ::64] = 7
    step = 2.0 ** torch.randint(-6, 2, (rows, cols // 64), generator=gen).float()
    v = (q.float().reshape(rows, -1, 64) * step.unsqueeze(-1)).reshape(rows, cols)
    return v, q.to(torch.int8), step.to(torch.float16)


def test_svdq_exact_on_the_grid_equals_matmul():
    """With x and the residual on the int4 grid, unit smoothing and a zero low-rank branch, the
    W4A4 product is numpy's matmul of the two matrices: a transposed, shifted or mis-scaled
    group fails it."""
    gen = torch.Generator().manual_seed(8)
    x, qx, sx = _on_grid(gen, 9, 320)
    w, qw, sw = _on_grid(gen, 24, 320)
    assert torch.equal(laws.int4_quantize(x)[0], qx) and torch.equal(laws.int4_quantize(x)[1], sx)
    codes, scales = laws.pack_int4(qw), sw
    down = torch.zeros(16, 320, dtype=torch.bfloat16)
    up = torch.zeros(24, 16, dtype=torch.bfloat16)
    got = laws.svdq_exact(x.to(torch.bfloat16), torch.ones(320), codes, scales, down, up, None)
    want = x.double().numpy() @ w.double().numpy().T
    assert np.array_equal(got.numpy(), want)
    bias = torch.randn(24, generator=gen).to(torch.bfloat16)
    got_b = laws.svdq_exact(x.to(torch.bfloat16), torch.ones(320), codes, scales, down, up, bias)
    assert np.array_equal(got_b.numpy(), want + bias.double().numpy())


def test_svdq_exact_low_rank_branch_only():
    """Zero residual codes: the product is the low-rank branch alone, bf16(x·downᵀ)·upᵀ."""
    gen = torch.Generator().manual_seed(9)
    x = torch.randint(-4, 5, (7, 128), generator=gen).to(torch.bfloat16)
    down = torch.randint(-3, 4, (32, 128), generator=gen).to(torch.bfloat16)
    up = torch.randint(-3, 4, (40, 32), generator=gen).to(torch.bfloat16)
    codes = torch.zeros(40, 64, dtype=torch.uint8)
    scales = torch.ones(40, 2, dtype=torch.float16)
    got = laws.svdq_exact(x, torch.ones(128), codes, scales, down, up, None)
    la = x.double().numpy() @ down.double().numpy().T  # small integers: exact in bf16
    assert np.array_equal(got.numpy(), la @ up.double().numpy().T)


def test_svdq_weight_reconstructs_effective_weight():
    """The producer's residual, dequantized and re-smoothed, plus up·down is W to within half a
    quantization step per element (the int4 round trip), and exactly W on the grid."""
    gen = torch.Generator().manual_seed(10)
    r, n, k = 16, 24, 192
    down = (torch.randn(r, k, generator=gen) * 0.02).to(torch.bfloat16)
    up = (torch.randn(n, r, generator=gen) * 0.02).to(torch.bfloat16)
    grid, _, _ = _on_grid(gen, n, k)
    p = 2.0 ** torch.randint(-1, 2, (k,), generator=gen).float()
    w = grid.double() * p.double() + up.double() @ down.double()
    codes, scales = laws.svdq_weight(w, p, down, up)
    deq = (laws.unpack_int4(codes).double().reshape(n, -1, 64) * scales.double().unsqueeze(-1)).reshape(n, k)
    assert np.allclose((deq * p.double() + up.double() @ down.double()).numpy(), w.numpy(), rtol=0, atol=1e-12)


# ------------------------------------------------------------------ svdq.nvfp4 (W4A4)

_E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def _nearest_even_e2m1(a: np.ndarray) -> np.ndarray:
    """Brute force: the index of the nearest E2M1 magnitude to each |a|, ties to the even index
    (the even mantissa), past 6 the top."""
    dist = np.abs(a[:, None] - _E2M1[None, :])
    best = dist.min(axis=1, keepdims=True)
    tied = dist == best
    idx = np.where(tied.sum(axis=1) > 1, np.argmax(tied & (np.arange(8) % 2 == 0), axis=1), np.argmin(dist, axis=1))
    return idx


def _unit_blocks(values: np.ndarray) -> torch.Tensor:
    """Blocks of 16 whose first element is 6 (amax 6 at g = 1: scale exactly 1), the other 15
    the values under test: |xs / (scale·g)| is then each value itself."""
    v = np.asarray(values, dtype=np.float32)
    pad = (-len(v)) % 15
    v = np.concatenate([v, np.zeros(pad, np.float32)]).reshape(-1, 15)
    blocks = np.concatenate([np.full((v.shape[0], 1), 6.0, np.float32), v], axis=1)
    return torch.from_numpy(blocks.reshape(1, -1))


def test_svdq_nvfp4_code_is_nearest_even_e2m1():
    """The threshold count of `svdq_nvfp4_quantize` against brute-force nearest-E2M1 with ties to
    the even code, on a dense sweep plus every midpoint and its float32 neighbours, both signs; a
    threshold with the wrong strictness fails at its midpoint."""
    mids = (_E2M1[:-1] + _E2M1[1:]) / 2
    near = np.concatenate([np.nextafter(mids.astype(np.float32), np.float32(0)), mids.astype(np.float32),
                           np.nextafter(mids.astype(np.float32), np.float32(7))])  # fmt: skip
    sweep = np.linspace(0, 6, 2401, dtype=np.float32)
    vals = np.concatenate([sweep, near]).astype(np.float32)
    xs = _unit_blocks(np.concatenate([vals, -vals]))
    codes, scales = laws.svdq_nvfp4_quantize(xs, torch.ones(1))
    assert (scales.float() == 1.0).all()
    got = codes.reshape(-1, 16)[:, 1:].reshape(-1).numpy()[: 2 * len(vals)]
    want = _nearest_even_e2m1(vals.astype(np.float64))
    assert np.array_equal(got[: len(vals)], want)
    neg = np.where(vals > 0, want + 8, want)  # -0 keeps code 0: the law's sign is xs < 0
    assert np.array_equal(got[len(vals):], neg)


def test_svdq_nvfp4_block_scale_and_saturation():
    """The block scale is the E4M3 encoding (independent bit encoder) of amax / (6g) clamped to
    [2^-9, 448]: all-zero blocks take the floor and code 0, a block past 448·6·g saturates its
    scale at 448 and its top elements at code 7."""
    gen = torch.Generator().manual_seed(21)
    xs = torch.randn(37, 256, generator=gen) * torch.exp2(torch.randint(-12, 12, (37, 1), generator=gen).float())
    xs[3] = 0
    xs[5, :16] = 448 * 6 * 40.0
    g = torch.tensor([0.0123])
    codes, scales = laws.svdq_nvfp4_quantize(xs, g)
    amax = xs.view(37, 16, 16).abs().amax(-1)
    ratio = (amax / (6.0 * g)).clamp(2.0**-9, 448.0)
    assert np.array_equal(scales.view(torch.uint8).numpy(), laws.e4m3_bits_numpy(ratio.numpy()))
    assert (scales[3].float() == 2.0**-9).all() and (codes[3] == 0).all()
    assert scales[5, 0].float() == 448.0 and (codes[5, :16] == 7).all()


def test_svdq_nvfp4_round_trip_bound():
    """Every element decodes to within half an E2M1 step (times scale·g) of xs, except past the
    top of a saturated block; the decoded block max is within the last step of amax."""
    gen = torch.Generator().manual_seed(22)
    x = torch.randn(64, 512, generator=gen).to(torch.bfloat16)
    p = torch.rand(512, generator=gen) + 0.5
    xs = laws.svdq_smooth(x, p)
    g = laws.svdq_nvfp4_input_scale(x, p)
    codes, scales = laws.svdq_nvfp4_quantize(xs, g)
    value = laws.svdq_nvfp4_values(codes, scales, g).double()
    unit = (scales.double() * g.double()).repeat_interleave(16, dim=1)
    a = (xs.double() / unit).abs()
    step = torch.where(a < 2, 0.5, torch.where(a < 4, 1.0, 2.0))
    assert ((value - xs.double()).abs() <= step / 2 * unit * (1 + 1e-6) + 1e-30).all()


def test_svdq_nvfp4_input_scale_brute_force():
    """g = fl(max over elements of fl(|x|·p)) / 2688, floored at 1e-30, element by element in
    numpy float32; a zero input gives the floor; a stored input_scale is returned as given."""
    gen = torch.Generator().manual_seed(23)
    for dtype in (torch.bfloat16, torch.float16):
        x = (torch.randn(9, 64, generator=gen) * 3).to(dtype)
        p = torch.rand(64, generator=gen) + 0.25
        xv, pv = x.float().numpy(), p.numpy()
        best = np.float32(0)
        for i in range(9):
            for j in range(64):
                best = max(best, np.float32(abs(xv[i, j])) * pv[j])
        want = max(np.float32(best) / np.float32(2688.0), np.float32(1e-30))
        got = laws.svdq_nvfp4_input_scale(x, p)
        assert got.numpy().view(np.uint32)[0] == np.float32(want).view(np.uint32)
    zero = laws.svdq_nvfp4_input_scale(torch.zeros(3, 64, dtype=torch.bfloat16), torch.ones(64))
    assert zero.item() == np.float32(1e-30)
    stored = torch.tensor(0.125)
    assert laws.svdq_nvfp4_input_scale(x, p, stored).item() == 0.125


def test_svdq_nvfp4_exact_on_the_grid_against_decode_law():
    """Activations already on the nvfp4 grid (amax 6 per block, stored g = 1, unit smoothing):
    quantization is lossless, and the W4A4 law equals x times the weight as the golden-pinned
    decode law (`decode_nvfp4`) decodes it, times c, plus the low-rank branch and the bias."""
    gen = torch.Generator().manual_seed(24)
    m, n, k, r = 5, 24, 128, 32
    codes = torch.randint(0, 16, (m, k), generator=gen).to(torch.uint8)
    codes[:, ::16] = 7
    codes[codes == 8] = 0  # -0 quantizes to code 0 (the law's sign is xs < 0)
    x = torch.tensor(laws.E2M1_VALUES)[codes.long()].to(torch.bfloat16)
    roles = {
        "weight": torch.randint(0, 256, (n, k // 2), generator=gen).to(torch.uint8),
        "scale": (torch.rand(n, k // 16, generator=gen) + 0.5).to(torch.float8_e4m3fn),
        "scale_2": torch.tensor([0.25]),
        "pre_quant_scale": torch.ones(k),
        "input_scale": torch.tensor(1.0),
        "channel_scale": torch.rand(n, generator=gen) + 0.5,
        "lowrank_down": torch.eye(k)[torch.randperm(k, generator=gen)[:r]].to(torch.bfloat16),
        "lowrank_up": (torch.randn(n, r, generator=gen) * 0.1).to(torch.bfloat16),
    }
    bias = torch.randn(n, generator=gen).to(torch.bfloat16)
    got_codes, got_scales = laws.svdq_nvfp4_quantize(laws.svdq_smooth(x, roles["pre_quant_scale"]), torch.ones(1))
    assert torch.equal(got_codes, codes) and (got_scales.float() == 1.0).all()
    w = laws.decode_nvfp4(roles["weight"], roles["scale"], roles["scale_2"], "row_major", False, False, None,
                          torch.float32).double()  # fmt: skip
    la = x.double() @ roles["lowrank_down"].double().t()  # one-hot rows: columns of x, exact in bf16
    want = (x.double() @ w.t()) * roles["channel_scale"].double() + la @ roles["lowrank_up"].double().t() + bias.double()
    assert torch.equal(laws.svdq_nvfp4_exact(x, roles, bias), want)


# ------------------------------------------------------------------- producer prologue


def test_prologue_norms_on_closed_forms():
    """A constant row c: RMS → c/√(c² + eps), layer → 0. An alternating row ±a: layer and RMS
    both → ±a/√(a² + eps). An identity prologue returns the rows widened."""
    c, a, eps = 3.0, 0.5, 1e-3
    const = torch.full((2, 256), c, dtype=torch.bfloat16)
    rms = laws.prologue(const, norm=laws.NORM_RMS, eps=eps)
    assert torch.allclose(rms, torch.full_like(rms, c / math.sqrt(c * c + eps)), rtol=2e-7)
    assert laws.prologue(const, norm=laws.NORM_LAYER, eps=eps).abs().max() == 0
    alt = torch.tensor([a, -a] * 128, dtype=torch.float16).repeat(3, 1)
    want = alt.double() / math.sqrt(a * a + eps)
    for norm in (laws.NORM_LAYER, laws.NORM_RMS):
        assert torch.allclose(laws.prologue(alt, norm=norm, eps=eps).double(), want, rtol=2e-7)
    x = torch.randn(5, 64, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    assert torch.equal(laws.prologue(x), x.float())


def test_prologue_modulation_tables_and_rows_per_entry():
    """scale −1 zeroes a row, scale 0 and shift 0 leave it; with zero rows and two table rows
    over four x rows, rows 0–1 read shift row 0 and rows 2–3 shift row 1."""
    gen = torch.Generator().manual_seed(2)
    x = torch.randn(4, 128, generator=gen).to(torch.bfloat16)
    assert laws.prologue(x, scale=torch.full((1, 128), -1.0, dtype=torch.bfloat16)).abs().max() == 0
    zeros = torch.zeros(2, 128, dtype=torch.bfloat16)
    assert torch.equal(laws.prologue(x, scale=zeros, shift=zeros), x.float())
    shift = torch.randn(2, 128, generator=gen).to(torch.bfloat16)
    got = laws.prologue(torch.zeros(4, 128, dtype=torch.bfloat16), shift=shift)
    assert torch.equal(got[:2], shift[:1].float().expand(2, -1))
    assert torch.equal(got[2:], shift[1:].float().expand(2, -1))


def test_prologue_activations_against_library_routines():
    """GELU (erf), tanh-GELU, SiTU and SwiGLU against Python's `math` routines in float64 (and
    torch's `silu`, the reference's eager SwiGLU), value by value."""
    vals = [-6.0, -2.5, -1.0, -0.25, 0.0, 0.125, 0.75, 1.5, 3.0, 8.0]
    x = torch.tensor([vals * 2], dtype=torch.float32).to(torch.bfloat16)
    xs = [float(v) for v in x.float().reshape(-1)]
    gelu = laws.prologue(x, activation=laws.ACT_GELU).reshape(-1)
    tanh_gelu = laws.prologue(x, activation=laws.ACT_GELU_TANH).reshape(-1)
    for got, v in zip(gelu.tolist(), xs):
        assert abs(got - 0.5 * v * (1 + math.erf(v / math.sqrt(2)))) <= 1e-6 * (1 + abs(v))
    for got, v in zip(tanh_gelu.tolist(), xs):
        want = 0.5 * v * (1 + math.tanh(0.79788456 * (v + 0.044715 * v**3)))
        assert abs(got - want) <= 1e-6 * (1 + abs(v))
    situ = laws.prologue(x, activation=laws.ACT_SITU).reshape(-1)  # h = first half, g = second
    half = len(xs) // 2
    for i, got in enumerate(situ.tolist()):
        h, g = xs[i], xs[half + i]
        want = 4 * math.tanh(g / 4) / (1 + math.exp(-g)) * 25 * math.tanh(h / 25)
        assert abs(got - want) <= 1e-5 * (1 + abs(want))
    ones = torch.ones_like(x)
    swiglu = laws.prologue(x, activation=laws.ACT_SWIGLU, up=ones)
    assert torch.equal(swiglu.to(torch.bfloat16), torch.nn.functional.silu(x.float()).to(torch.bfloat16))
    halves = laws.prologue(torch.cat([ones, x], -1), activation=laws.ACT_SWIGLU)
    assert torch.equal(halves, swiglu)


# ------------------------------------------------------------------------------ w4a8


def _e4m3_bytes(values: list[int]) -> torch.Tensor:
    return torch.tensor(values, dtype=torch.uint8).view(torch.float8_e4m3fn)


def test_w4a8_unpack_closed_forms():
    """Scale byte 0x38 (1.0) on the uniform grid gives q − 8; byte i holds k = 2i in its low
    nibble; NaN scales (0x7F, 0xFF) level to 0; 448 (0x7E) times the codebook's ±0.98 clamps to
    ±127."""
    codes = torch.tensor([[0x10 * (2 * i + 1 & 15) + (2 * i & 15) for i in range(8)]], dtype=torch.uint8)
    one = _e4m3_bytes([0x38]).reshape(1, 1)
    got = laws.w4a8_unpack(codes, one, None)
    assert got.tolist() == [[k - 8 for k in range(16)]]
    nan = _e4m3_bytes([0x7F]).reshape(1, 1)
    assert laws.w4a8_unpack(codes, nan, None).abs().max() == 0
    book = torch.tensor(laws.W4A8_CODEBOOK)
    big = laws.w4a8_unpack(codes, _e4m3_bytes([0x7E]).reshape(1, 1), book)
    assert big[0, 0] == -127 and big[0, 15] == 127


def test_w4a8_unpack_every_scale_and_code_against_numpy():
    """Every (E4M3 scale byte, code) pair, codebook and uniform grid: the float32 product
    rounded half to even (numpy's float32 multiply and `rint`), NaN to 0, clamped to ±127."""
    codes = torch.tensor([[0x10 * (2 * i + 1) + 2 * i for i in range(8)]] * 256, dtype=torch.uint8)
    scales = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).reshape(256, 1)
    scale_f = np.array([[float(v)] for v in scales.float().reshape(-1)], dtype=np.float32)
    for book in (torch.tensor(laws.W4A8_CODEBOOK), None):
        levels = np.arange(-8, 8, dtype=np.float32) if book is None else book.numpy().astype(np.float32)
        with np.errstate(invalid="ignore"):
            want = np.rint(scale_f * levels[None, :])
        want = np.clip(np.nan_to_num(want, nan=0.0), -127, 127).astype(np.int8)
        assert np.array_equal(laws.w4a8_unpack(codes, scales, book).numpy(), want)


def test_svdq_nvfp4_nan_block_is_pinned():
    """A block holding a NaN under `svdq_nvfp4_quantize`, against what IEEE arithmetic fixes: its
    amax is NaN, so its scale is the E4M3 NaN byte 0x7F; every quotient by a NaN scale is NaN and
    fails every threshold comparison, so each code is 0, + 8 where the element is negative (the
    NaN itself is not); a neighbouring block is as without the NaN. The input scale of a tensor
    holding a NaN is NaN (amax and clamp propagate it)."""
    xs = torch.zeros(1, 32)
    xs[0, :16] = torch.linspace(-3, 3, 16)
    xs[0, 16:] = torch.linspace(-3, 3, 16)
    xs[0, 5] = float("nan")
    g = torch.tensor([0.5])
    codes, scales = laws.svdq_nvfp4_quantize(xs, g)
    assert scales.view(torch.uint8)[0, 0] == 0x7F
    want = (xs[0, :16] < 0).to(torch.uint8) * 8
    assert torch.equal(codes[0, :16], want)
    clean = xs.clone()
    clean[0, :16] = 0
    c2, s2 = laws.svdq_nvfp4_quantize(clean, g)
    assert torch.equal(codes[0, 16:], c2[0, 16:]) and scales[0, 1].view(torch.uint8) == s2[0, 1].view(torch.uint8)
    assert torch.isnan(laws.svdq_nvfp4_input_scale(xs, torch.ones(32))).all()

"""GPU parity of the SVDQuant W4A4 (int4-g64) kernels against the CPU oracle, through the C ABI.

Bar: packed int4 codes and fp16 group scales bit-exact to `laws.int4_quantize(laws.svdq_smooth(..))`;
the low-rank input la = bf16(x·downᵀ) within one bf16 step of the exactly summed value (the
kernel sums in float32, the oracle exactly); outputs within |got − exact| ≤ ATOL·rms(exact) +
RTOL·|exact| of the float64 W4A4 product (`laws.svdq_exact`).
"""

from __future__ import annotations

import pytest
import torch

from fullsize import tile_rows
from oracle import laws

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-2, 2e-2
DEV = "cuda:0"


@pytest.fixture(scope="module")
def ops():
    from cozyq import prebuilt

    return prebuilt.library(0)


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def activations(m: int, k: int, seed: int, dtype=torch.bfloat16) -> torch.Tensor:
    """~N(0,1) with 1% of the channels scaled x20."""
    gen = _gen(seed)
    x = torch.randn(m, k, generator=gen)
    chans = torch.randperm(k, generator=gen)[: max(1, k // 100)]
    x[:, chans] *= 20
    return x.to(dtype)


def operands(n: int, k: int, r: int, seed: int):
    """The C4 recipe: smoothing p ~ U[0.5, 2], down [R, K] and up [N, R] ~ N(0, 0.02) in bf16,
    W ~ N(0, 0.02), residual quantized by the build's producer."""
    gen = _gen(seed)
    p = torch.rand(k, generator=gen) * 1.5 + 0.5
    down = (torch.randn(r, k, generator=gen) * 0.02).to(torch.bfloat16)
    up = (torch.randn(n, r, generator=gen) * 0.02).to(torch.bfloat16)
    w = torch.randn(n, k, generator=gen) * 0.02
    codes, scales = laws.svdq_weight(w, p, down, up)
    return p, down, up, codes, scales


def assert_close(got: torch.Tensor, exact: torch.Tensor) -> None:
    got, exact = got.double().cpu(), exact.double().cpu()
    rms = exact.pow(2).mean().sqrt().item()
    bound = ATOL * rms + RTOL * exact.abs()
    err = (got - exact).abs()
    worst = (err - bound).max().item()
    assert worst <= 0, f"max excess {worst:.3g} (rms {rms:.3g}, max err {err.max().item():.3g})"


def assert_la(got: torch.Tensor, x: torch.Tensor, down: torch.Tensor) -> None:
    """Within one bf16 step of x·downᵀ summed exactly (and bit-equal to its rounding almost
    everywhere)."""
    half = x.dtype
    exact = x.to(half).double() @ down.to(half).double().t()
    want = exact.to(torch.bfloat16)
    got = got.cpu()
    step = (want.float().abs() * 2.0 ** -7).clamp(min=2.0 ** -133).double()
    assert ((got.double() - exact).abs() <= step).all()
    assert (got != want).double().mean().item() < 0.02


@pytest.mark.parametrize("rank", [16, 32, 64])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(1, 64), (5, 192), (77, 3072), (300, 1024), (3, 12352)],
                         ids=lambda s: f"{s[0]}x{s[1]}")  # fmt: skip
def test_svdq_quantize_bit_exact(ops, shape, dtype, rank):
    m, k = shape
    x = activations(m, k, 31 + m, dtype)
    p, down, _, _, _ = operands(8, k, rank, 32 + k)
    act, ascales, la = ops.svdq_int4_quantize(x.to(DEV), p.to(DEV), down.to(DEV))
    torch.cuda.synchronize()
    q, s = laws.int4_quantize(laws.svdq_smooth(x, p))
    assert torch.equal(act.cpu(), laws.pack_int4(q))
    assert torch.equal(ascales.cpu().view(torch.int16), s.view(torch.int16))
    assert_la(la, x, down)


def test_svdq_quantize_edge_groups(ops):
    """A zero group (scale 0, codes 0), a group whose amax/7 overflows fp16 (scale inf, codes 0),
    and one whose scale is an fp16 subnormal."""
    k = 256
    x = activations(4, k, 41)
    x[0, 64:128] = 0
    x[1, 0:64] = 1.0e6
    x[2, 128:192] = (torch.randn(64) * 1e-6).to(torch.bfloat16)
    p, down, _, _, _ = operands(8, k, 16, 42)
    act, ascales, la = ops.svdq_int4_quantize(x.to(DEV), p.to(DEV), down.to(DEV))
    torch.cuda.synchronize()
    q, s = laws.int4_quantize(laws.svdq_smooth(x, p))
    assert s[0, 1] == 0 and torch.isinf(s[1, 0]) and 0 < float(s[2, 2]) < 6.1e-5
    assert torch.equal(act.cpu(), laws.pack_int4(q))
    assert torch.equal(ascales.cpu().view(torch.int16), s.view(torch.int16))
    assert_la(la, x, down)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("shape", [(77, 136, 192, 16), (300, 256, 1024, 32), (128, 384, 3072, 64),
                                   (1, 8, 64, 32), (260, 520, 320, 32)],
                         ids=lambda s: "x".join(map(str, s)))  # fmt: skip
def test_svdq_linear_within_tolerance(ops, shape, bias, out_dtype):
    m, n, k, r = shape
    x = activations(m, k, 51 + m)
    p, down, up, codes, scales = operands(n, k, r, 52 + n)
    b = (torch.randn(n, generator=_gen(53)) * 0.5).to(out_dtype) if bias else None
    out = ops.svdq_int4_linear(x.to(DEV), p.to(DEV), down.to(DEV), codes.to(DEV), scales.to(DEV),
                          up.to(DEV), None if b is None else b.to(DEV), out_dtype)  # fmt: skip
    torch.cuda.synchronize()
    assert out.dtype == out_dtype and out.shape == (m, n)
    assert_close(out, laws.svdq_exact(x, p, codes, scales, down, up, b))


def test_svdq_gemm_on_oracle_operands(ops):
    """The GEMM alone, fed the oracle's own codes, scales and la: isolates the product from the
    activation kernel."""
    m, n, k, r = 200, 264, 640, 32
    x = activations(m, k, 61)
    p, down, up, codes, scales = operands(n, k, r, 62)
    q, s = laws.int4_quantize(laws.svdq_smooth(x, p))
    la = laws.svdq_down(x, down)
    out = ops.svdq_int4_gemm(laws.pack_int4(q).to(DEV), s.to(DEV), la.to(DEV), codes.to(DEV),
                        scales.to(DEV), up.to(DEV), None, torch.bfloat16)  # fmt: skip
    torch.cuda.synchronize()
    assert_close(out, laws.svdq_exact(x, p, codes, scales, down, up, None))


def test_svdq_c4_full_size_sampled_rows(ops):
    """Config 4 at its full size (M=4096, K=N=3072, R=32): every code and scale bit-exact, and 4
    rows of every M-tile (64, each against every column) within tolerance."""
    m, n, k, r = 4096, 3072, 3072, 32
    x = activations(m, k, 20261205)
    p, down, up, codes, scales = operands(n, k, r, 20261206)
    bias = (torch.randn(n, generator=_gen(7)) * 0.5).to(torch.bfloat16)
    xd = x.to(DEV)
    act, ascales, la = ops.svdq_int4_quantize(xd, p.to(DEV), down.to(DEV))
    out = ops.svdq_int4_gemm(act, ascales, la, codes.to(DEV), scales.to(DEV), up.to(DEV), bias.to(DEV),
                        torch.bfloat16)  # fmt: skip
    torch.cuda.synchronize()
    q, s = laws.int4_quantize(laws.svdq_smooth(x, p))
    assert torch.equal(act.cpu(), laws.pack_int4(q))
    assert torch.equal(ascales.cpu().view(torch.int16), s.view(torch.int16))
    rows = tile_rows(m)
    assert_close(out.cpu()[rows], laws.svdq_exact(x[rows], p, codes, scales, down, up, bias))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["f32", "bf16", "fp16"])
@pytest.mark.parametrize("shape", [(3072, 3072, 32), (264, 1024, 16), (2, 64, 64), (40, 320, 0)],
                         ids=lambda s: "x".join(map(str, s)))  # fmt: skip
def test_svdq_int4_weight_encoder_bit_exact(shape, dtype):
    """`encode.encode_svdq_int4` (the HIP producer the C4 bench builds its weight with) gives the
    oracle producer's codes and fp16 scales bit for bit, from f32, bf16 and fp16 sources, with an
    all-zero group (scale 0, codes 0) and rank 0; its measured loss is the dense decode's."""
    from cozyq import encode

    n, k, r = shape
    gen = _gen(n + k + r)
    w = (torch.randn(n, k, generator=gen) * 0.02).to(dtype)
    w[0, :64] = 0
    p = torch.rand(k, generator=gen) * 1.5 + 0.5
    down = (torch.randn(r, k, generator=gen) * 0.02).to(torch.bfloat16)
    up = (torch.randn(n, r, generator=gen) * 0.02).to(torch.bfloat16)
    if r:
        up[0] = 0  # row 0's first group stays all zero
    enc = encode.encode_svdq_int4(torch, "w", w.to(DEV), p, down, up)
    codes, scales = laws.svdq_weight(w.float(), p, down, up)
    assert torch.equal(enc.payload.cpu(), codes)
    assert torch.equal(enc.companions[0].raw.cpu().view(torch.int16), scales.view(torch.int16))
    assert (enc.companions[0].raw[0, 0] == 0).item()
    assert enc.energy > 0 and 0 < enc.relative_frobenius() < 0.2

"""The weight encoders (`cozyq.encode`, kernels in `csrc/encode.hip`).

The reference's producers live in tensorfs (`derive/microscale.py:146-408`), whose arithmetic is
not in the reference, so the laws are this build's: the oracle restates each (`oracle/laws.py`),
and the CPU tests below pin the restatements by closed forms and brute force. The GPU tests hold
the kernels bit-exact to the oracle on float32, bf16 and fp16 inputs, and the measured facts
(sse, energy, max |error|) to float64 sums over the oracle's decode.
"""

from __future__ import annotations

import pytest
import torch

from oracle import laws

# ----------------------------------------------------------------------- CPU: the laws


def test_e2m1_code_rounds_to_nearest_even_and_saturates():
    grid = torch.tensor(laws.E2M1_VALUES[:8])
    # every grid point maps to itself
    assert torch.equal(laws.e2m1_code(grid), torch.arange(8, dtype=torch.int32))
    # midpoints go to the even code; past 6 saturates
    mids = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 7.0, 1e9])
    assert laws.e2m1_code(mids).tolist() == [0, 2, 2, 4, 4, 6, 6, 7, 7]
    # nearest by brute force away from ties, sign in bit 3
    x = torch.linspace(-6.5, 6.5, 2601)
    codes = laws.e2m1_code(x)
    values = torch.tensor(laws.E2M1_VALUES)[codes.long()]
    best = (grid.view(1, -1) - x.abs().clamp(max=6).view(-1, 1)).abs().min(dim=1).values
    assert torch.allclose((values.abs() - x.abs().clamp(max=6)).abs(), best)
    assert bool(((codes >= 8) == (x < 0)).all())


def test_nvfp4_encoder_closed_forms():
    # An all-zero matrix: g = 1, zero scales and codes.
    packed, scale, g, sat = laws.encode_nvfp4(torch.zeros(2, 32))
    assert float(g) == 1.0 and int(packed.sum()) == 0 and int(scale.sum()) == 0 and sat == 0
    # Blocks built from grid values times an E4M3 scale times g decode exactly.
    g_true = 448.0 * 6.0  # amax 6·448·g / 2688 -> g = amax / 2688
    codes = torch.randint(0, 16, (4, 64))
    s = torch.tensor([1.0, 2.0, 0.5, 448.0]).repeat_interleave(64).view(4, 64)
    w = torch.tensor(laws.E2M1_VALUES)[codes] * s
    w[:, 0] = 6.0 * s[:, 0]  # every block holds its maximum, so c0 is the exact scale
    w[:, 16] = 6.0 * s[:, 16]
    w[:, 32] = 6.0 * s[:, 32]
    w[:, 48] = 6.0 * s[:, 48]
    packed, scale, g, sat = laws.encode_nvfp4(w)
    back = laws.decode_nvfp4(packed, scale.view(torch.float8_e4m3fn), g, "row_major", False, False,
                             None, torch.float32)  # fmt: skip
    assert float(g) == float(w.abs().max()) / g_true
    assert torch.equal(back, w) and sat == 0


def test_nvfp4_encoder_picks_the_least_error_candidate():
    """Brute force: the chosen E4M3 scale is one of c0 − 1, c0, c0 + 1 (c0 the block maximum's
    scale) and none of those decodes the block with less squared error."""
    torch.manual_seed(1)
    w = torch.randn(16, 256)
    packed, scale, g, _ = laws.encode_nvfp4(w)
    blocks = w.view(16, 16, 16)
    lut = torch.tensor(laws.E2M1_VALUES)

    def err(code: torch.Tensor) -> torch.Tensor:
        s = code.to(torch.uint8).view(torch.float8_e4m3fn).float().unsqueeze(-1)
        d = s * g
        q = laws.e2m1_code(blocks / d)
        diff = blocks - (lut[q.long()] * s) * g
        total = torch.zeros(16, 16)
        for k in range(16):
            total = total + diff[..., k] * diff[..., k]
        return total

    c0 = (blocks.abs().amax(-1) / (6.0 * g)).to(torch.float8_e4m3fn).view(torch.uint8).to(torch.int32)
    chosen = scale.to(torch.int32)
    assert bool(((chosen - c0).abs() <= 1).all())
    for delta in (-1, 0, 1):
        assert bool((err(chosen) <= err((c0 + delta).clamp(1, 0x7E))).all())


def test_w4a8_encoder_codes_are_the_nearest_levels():
    """Brute force over every code: the unpacked level of each element is the closest of the 16
    levels to its target t = r/s."""
    torch.manual_seed(2)
    w = torch.randn(4, 512) * 0.02
    codes, group, scale = laws.encode_w4a8(w)
    cb = torch.tensor(laws.W4A8_CODEBOOK)
    levels = laws.w4a8_unpack(codes, group.view(torch.float8_e4m3fn), cb).float()
    r = laws.hadamard(w.float(), 256).mul_(1.0 / 16)
    t = r / scale.unsqueeze(-1)
    sigma = group.view(torch.float8_e4m3fn).float().repeat_interleave(16, dim=1)
    every = torch.round(cb.view(1, 1, 16) * sigma.unsqueeze(-1)).clamp(-127, 127)
    best = (every - t.unsqueeze(-1)).abs().min(dim=-1).values
    assert torch.equal((levels - t).abs(), best)
    # the group scale covers the group: max|t| / max|c| rounded to E4M3
    ga = t.view(4, -1, 16).abs().amax(-1)
    assert torch.equal(group.view(torch.float8_e4m3fn), (ga / cb.abs().max()).to(torch.float8_e4m3fn))


def test_w4a8_encoder_is_exact_on_its_own_levels():
    """Rows whose rotated, scaled values are exactly codebook levels encode without loss in the
    int8 domain: decoding gives back (H·levels)·s/16."""
    torch.manual_seed(3)
    cb = torch.tensor(laws.W4A8_CODEBOOK)
    # choose int8-domain targets on levels of σ = 127/0.980671 rounded to E4M3 (= 128)
    sigma = torch.tensor(127.0 / 0.980671).to(torch.float8_e4m3fn).float()
    lv = torch.round(cb * sigma).clamp(-127, 127)
    pick = torch.randint(0, 16, (2, 256))
    pick[:, ::16] = 15  # each group holds the top level, so σ comes back the same
    t = lv[pick]
    s = torch.tensor([0.01, 0.003])
    r = t * s.unsqueeze(-1)
    w = laws.hadamard(r, 256).mul_(1.0 / 16)  # H·H = 256·I: rotating back
    codes, group, scale = laws.encode_w4a8(w)
    got = laws.w4a8_unpack(codes, group.view(torch.float8_e4m3fn), cb).float()
    assert torch.allclose(got, t)


# ----------------------------------------------------------------------- GPU: the kernels

CUDA = "cuda:0"
DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _weights(rows: int, cols: int, dtype: torch.dtype, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(rows, cols, generator=g) * 0.02
    w[:, torch.randperm(cols, generator=g)[: max(1, cols // 100)]] *= 20
    return w.to(dtype)


def _encode():
    from cozyq import encode

    return encode


def _facts(w: torch.Tensor, decoded: torch.Tensor) -> tuple[float, float, float]:
    x, y = w.double(), decoded.double()
    return float(((x - y) ** 2).sum()), float((x * x).sum()), float((x - y).abs().max())


def _check_facts(enc, w: torch.Tensor, decoded: torch.Tensor) -> None:
    sse, energy, worst = _facts(w, decoded)
    assert enc.sse == pytest.approx(sse, rel=1e-9, abs=1e-30)
    assert enc.energy == pytest.approx(energy, rel=1e-9)
    assert enc.max_abs_err == pytest.approx(worst, rel=1e-12, abs=0)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(300, 3072), (64, 256), (5, 12288)])
def test_gpu_int8_convrot_encoder(dtype, shape):
    encode = _encode()
    w = _weights(*shape, dtype, 1)
    enc = encode.encode_int8_convrot256(torch, "w", w.to(CUDA))
    q, s = laws.int8_weight_rotated(w, 256)
    assert torch.equal(enc.payload.cpu(), q)
    assert torch.equal(enc.companions[0].raw.cpu(), s)
    _check_facts(enc, w, laws.decode_int8_convrot(q, s, 256, torch.float32))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(300, 3072), (7, 4104)])
def test_gpu_fp8_rowwise_encoder(dtype, shape):
    encode = _encode()
    w = _weights(*shape, dtype, 2)
    enc = encode.encode_fp8_rowwise(torch, "w", w.to(CUDA))
    q, s = laws.fp8_weight(w)
    assert torch.equal(enc.payload.cpu().view(torch.uint8), q.view(torch.uint8))
    assert torch.equal(enc.companions[0].raw.cpu(), s)
    _check_facts(enc, w, laws.decode_rowwise(q, s, torch.float32))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("layout", ["row_major", "cublas_128x4"])
def test_gpu_mxfp8_encoder(dtype, layout):
    encode = _encode()
    w = _weights(300, 1024, dtype, 3)
    enc = encode.encode_mxfp8(torch, "w", w.to(CUDA), layout)
    q, b = laws.mx_quantize(w)
    assert torch.equal(enc.payload.cpu().view(torch.uint8), q.view(torch.uint8))
    grid = enc.companions[0].raw.cpu()
    if layout == "cublas_128x4":
        assert torch.equal(laws.to_blocked(b), grid.reshape(-1))
    else:
        assert torch.equal(grid, b)
    _check_facts(enc, w, laws.mx_dequantize(q, b))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(300, 3072), (33, 512)])
def test_gpu_w4a8_encoder(dtype, shape):
    encode = _encode()
    w = _weights(*shape, dtype, 4)
    enc = encode.encode_w4a8(torch, "w", w.to(CUDA))
    codes, group, scale = laws.encode_w4a8(w)
    assert torch.equal(enc.payload.cpu(), codes)
    assert torch.equal(enc.companions[0].raw.cpu().view(torch.uint8), group)
    assert torch.equal(enc.companions[1].raw.cpu(), scale)
    cb = torch.tensor(laws.W4A8_CODEBOOK)
    levels = laws.w4a8_unpack(codes, group.view(torch.float8_e4m3fn), cb)
    _check_facts(enc, w, laws.decode_int8_convrot(levels, scale, 256, torch.float32))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(300, 3072), (3, 48)])
def test_gpu_nvfp4_encoder(dtype, shape):
    encode = _encode()
    w = _weights(*shape, dtype, 5)
    enc = encode.encode_nvfp4(torch, "w", w.to(CUDA))
    packed, scale, g, sat = laws.encode_nvfp4(w)
    assert torch.equal(enc.payload.cpu(), packed)
    assert torch.equal(enc.companions[0].raw.cpu().view(torch.uint8), scale)
    assert float(enc.companions[1].raw.cpu()) == float(g)
    assert enc.saturated == sat
    decoded = laws.decode_nvfp4(packed, scale.view(torch.float8_e4m3fn), g, "row_major", False,
                                False, None, torch.float32)  # fmt: skip
    _check_facts(enc, w, decoded)
    assert 0.0 < enc.relative_frobenius() < 0.2


@pytest.mark.gpu
def test_gpu_encoders_refuse_like_the_reference():
    encode = _encode()
    with pytest.raises(encode.UnsupportedInput, match="multiple of the 256-element block"):
        encode.encode_int8_convrot256(torch, "w", torch.zeros(2, 100, device=CUDA))
    with pytest.raises(encode.UnsupportedInput, match="rank 1"):
        encode.encode_nvfp4(torch, "w", torch.zeros(64, device=CUDA))
    bad = torch.zeros(2, 256, device=CUDA)
    bad[1, 3] = float("inf")
    with pytest.raises(encode.UnsupportedInput, match="non-finite"):
        encode.encode_w4a8(torch, "w", bad)

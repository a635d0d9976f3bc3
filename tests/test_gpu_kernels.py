"""GPU parity of the HIP kernels against the CPU oracle (`oracle/laws.py`), through the C ABI.

Bar: codes, scales and int32 accumulators bit-exact; int8 outputs bit-exact to the CPU law
(`internal/int8_linear.py:431-448` + `:276`); fp8, MXFP8 and GELU outputs within
|got − exact| ≤ ATOL·rms(exact) + RTOL·|exact| of the float64 product of the law's codes.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from fullsize import checksums_exact, tile_rows
from oracle import laws

pytestmark = pytest.mark.gpu

#: Output tolerance for float-accumulated products: atol relative to the output RMS, and rtol.
ATOL, RTOL = 1e-2, 2e-2
DEV = "cuda:0"


@pytest.fixture(scope="module")
def ops():
    from cozyq import prebuilt

    return prebuilt.library(0)


def activations(m: int, k: int, seed: int, dtype=torch.bfloat16) -> torch.Tensor:
    """~N(0,1) with 1% of the channels scaled x20 (the BASELINE outlier distribution)."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=gen)
    chans = torch.randperm(k, generator=gen)[: max(1, k // 100)]
    x[:, chans] *= 20
    return x.to(dtype)


def weights(n: int, k: int, seed: int) -> torch.Tensor:
    gen = torch.Generator().manual_seed(seed)
    return torch.randn(n, k, generator=gen) * 0.02


def assert_close(got: torch.Tensor, exact: torch.Tensor) -> None:
    got, exact = got.double().cpu(), exact.double().cpu()
    rms = exact.pow(2).mean().sqrt().item()
    bound = ATOL * rms + RTOL * exact.abs()
    err = (got - exact).abs()
    worst = (err - bound).max().item()
    assert worst <= 0, f"max excess {worst:.3g} (rms {rms:.3g}, max err {err.max().item():.3g})"


# --------------------------------------------------------- hardware E4M3 conversion


def test_hardware_e4m3_conversion_matches_torch_cast():
    """gfx950's v_cvt_pk_fp8_f32 against torch's `.to(float8_e4m3fn)` (via the software encoder,
    itself held to torch's cast in test_abi) on every float32 within ±448 at a stride of 61
    patterns, every float32 in [2^-11, 2^-5] (the subnormal boundary), and every E4M3 rounding
    midpoint ±2 ulp, both signs: the quantizers use it only if all agree."""
    from cozyq import _lib

    lib = _lib.load()
    top = int(np.float32(448.0).view(np.uint32))
    sweep = np.arange(0, top + 1, 61, dtype=np.uint32)
    low = np.arange(np.float32(2.0**-11).view(np.uint32), np.float32(2.0**-5).view(np.uint32),
                    dtype=np.uint32)  # fmt: skip
    codes = np.arange(0, 0x7F, dtype=np.uint8)
    vals = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32).view(np.uint32).astype(np.int64)
    near = np.clip(np.concatenate([mids + d for d in (-2, -1, 0, 1, 2)]), 0, None).astype(np.uint32)
    bits = np.concatenate([sweep, low, near, np.array([top], np.uint32)])
    v = bits.view(np.float32)
    v = np.concatenate([v, -v])
    if v.size % 2:
        v = v[:-1]
    want = np.zeros(v.shape, dtype=np.uint8)
    lib.cozyq_host_e4m3(v.ctypes.data, want.ctypes.data, v.size)
    tin = torch.from_numpy(v).to(DEV)
    tout = torch.empty(v.size, dtype=torch.uint8, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.cozyq_probe_e4m3(0, tin.data_ptr(), tout.data_ptr(), v.size, stream) == 0
    got = tout.cpu().numpy()
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} differ, e.g. {v[bad[:4]]} -> {got[bad[:4]]} vs {want[bad[:4]]}"


def test_reciprocal_division_matches_ieee_division():
    """div_rn (q = x·RN(1/s), one FMA correction) against correctly rounded float32 division on
    100M pairs with random significands and exponents spanning ±60 binades: bit-identical
    wherever the quotient is a normal float (an underflowing quotient only has to stay tiny:
    every caller maps it to code 0)."""
    from cozyq import _lib

    lib = _lib.load()
    gen = torch.Generator(device=DEV).manual_seed(17)
    n = 100_000_000
    mant = torch.rand(n, generator=gen, device=DEV) + 1.0
    x = mant * torch.exp2(torch.randint(-60, 61, (n,), generator=gen, device=DEV).float())
    x = torch.where(torch.rand(n, generator=gen, device=DEV) < 0.5, -x, x)
    x[:1000] = 0.0
    x[1000:2000] = -0.0  # a signed zero keeps its sign: e4m3 codes it 0x80
    s = (torch.rand(n, generator=gen, device=DEV) + 1.0) * torch.exp2(
        torch.randint(-60, 61, (n,), generator=gen, device=DEV).float())
    out = torch.empty_like(x)
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.cozyq_probe_div(0, x.data_ptr(), s.data_ptr(), out.data_ptr(), n, stream) == 0
    want = x.cpu() / s.cpu()  # IEEE float32 division on the host
    got = out.cpu()
    normal = want.abs() >= 2.0**-126
    assert torch.equal(got[normal], want[normal])
    assert (got[~normal].abs() < 2.0**-100).all()
    assert torch.equal(torch.signbit(got), torch.signbit(want))


# ---------------------------------------------------------------------- MFMA layouts


def _probe(kind: int, a: np.ndarray, b: np.ndarray, sa=None, sb=None) -> np.ndarray:
    from cozyq import _lib

    lib = _lib.load()
    ta = torch.from_numpy(a.view(np.uint8).reshape(64, 32)).to(DEV)
    tb = torch.from_numpy(b.view(np.uint8).reshape(64, 32)).to(DEV)
    tsa = torch.from_numpy(np.zeros(64, np.uint8) if sa is None else sa).to(DEV)
    tsb = torch.from_numpy(np.zeros(64, np.uint8) if sb is None else sb).to(DEV)
    d = torch.zeros(64, 16, dtype=torch.int32, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    code = lib.cozyq_probe_mfma(0, kind, ta.data_ptr(), tb.data_ptr(), tsa.data_ptr(),
                                tsb.data_ptr(), d.data_ptr(), stream)  # fmt: skip
    assert code == 0
    torch.cuda.synchronize()
    out = d.cpu().numpy()
    return out if kind in (4, 5, 6, 7, 8) else out[:, :4].copy()


def _expand(lanes: np.ndarray, per_lane: int) -> np.ndarray:
    """Per-lane slices -> the 16 x (4·per_lane) matrix they stand for: lane l supplies row l%16,
    K slice l//16."""
    mat = np.zeros((16, 4 * per_lane), dtype=lanes.dtype)
    for lane in range(64):
        mat[lane % 16, (lane // 16) * per_lane:(lane // 16 + 1) * per_lane] = lanes[lane]
    return mat


def _check_layout(d: np.ndarray, want: np.ndarray, exact: bool) -> None:
    for lane in range(64):
        for r in range(4):
            got, ref = d[lane, r], want[4 * (lane // 16) + r, lane % 16]
            if exact:
                assert got == ref, (lane, r)
            else:
                assert abs(got - ref) <= 1e-5 * (1 + abs(ref)), (lane, r, got, ref)


def test_mfma_i8_layout():
    rng = np.random.default_rng(0)
    a = rng.integers(-128, 128, (64, 32), dtype=np.int8)
    b = rng.integers(-128, 128, (64, 32), dtype=np.int8)
    d = _probe(0, a, b).astype(np.int64)
    want = _expand(a[:, :16], 16).astype(np.int64) @ _expand(b[:, :16], 16).astype(np.int64).T
    _check_layout(d, want, exact=True)


def test_mfma_i8_32x32_layout():
    """32x32x32: lane l supplies row (column) l%32 and K chunk l/32; result register r of lane l
    is row 8·(r/4) + 4·(l/32) + r%4 of column l%32."""
    rng = np.random.default_rng(5)
    a = rng.integers(-128, 128, (64, 32), dtype=np.int8)
    b = rng.integers(-128, 128, (64, 32), dtype=np.int8)
    d = _probe(4, a, b).astype(np.int64)

    def expand(lanes):
        mat = np.zeros((32, 32), dtype=np.int64)
        for lane in range(64):
            mat[lane % 32, 16 * (lane // 32):16 * (lane // 32) + 16] = lanes[lane, :16]
        return mat

    want = expand(a) @ expand(b).T
    for lane in range(64):
        for r in range(16):
            assert d[lane, r] == want[8 * (r // 4) + 4 * (lane // 32) + r % 4, lane % 32], (lane, r)


def _e4m3_lanes(rng) -> np.ndarray:
    codes = rng.integers(0, 256, (64, 32), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x38  # no NaN codes
    return codes


def _e4m3_values(codes: np.ndarray) -> np.ndarray:
    return torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).double().numpy()


def _f8_matrix(lanes: np.ndarray, scales: np.ndarray | None = None) -> np.ndarray:
    """The 16 x 128 operand the f8f6f4 MFMA reads from 64 lanes x 32 bytes: lane group g holds
    k in [16g, 16g+16) in bytes 0..15 and k in [64+16g, 80+16g) in bytes 16..31; the E8M0 byte
    of row i's K block κ (k in [32κ, 32κ+32)) is lane i + 16κ's."""
    mat = np.zeros((16, 128))
    for lane in range(64):
        i, g = lane % 16, lane // 16
        mat[i, 16 * g:16 * g + 16] = lanes[lane, :16]
        mat[i, 64 + 16 * g:80 + 16 * g] = lanes[lane, 16:]
    if scales is not None:
        for i in range(16):
            for kb in range(4):
                mat[i, 32 * kb:32 * kb + 32] *= 2.0 ** (float(scales[i + 16 * kb]) - 127)
    return mat


#: The f8f6f4 matrix core's sum of 128 exact e4m3 products is not a sequential float32 sum:
#: measured on gfx950 within 2^-14.6 of the sum of the products' magnitudes; held to 2^-13.
F8_SUM_BOUND = 2.0 ** -13


def _check_f8(d: np.ndarray, a: np.ndarray, b: np.ndarray, bound: float = F8_SUM_BOUND) -> None:
    want = a @ b.T
    size = np.abs(a) @ np.abs(b).T
    for lane in range(64):
        for r in range(4):
            i, j = 4 * (lane // 16) + r, lane % 16
            err = abs(d[lane, r] - want[i, j])
            assert err <= bound * size[i, j] + 1e-30, (lane, r, err / size[i, j])


def test_mfma_f8_layout():
    rng = np.random.default_rng(1)
    a, b = _e4m3_lanes(rng), _e4m3_lanes(rng)
    d = _probe(1, a, b).view(np.float32).astype(np.float64)
    _check_f8(d, _f8_matrix(_e4m3_values(a)), _f8_matrix(_e4m3_values(b)))


def test_mfma_f8_scaled_layout():
    """Each lane's E8M0 byte scales one 32-element K block of one row (column). With scales the
    matrix core's sum is coarser still: measured within 2^-12.9 of the magnitudes' sum."""
    rng = np.random.default_rng(2)
    a, b = _e4m3_lanes(rng), _e4m3_lanes(rng)
    sa = rng.integers(118, 136, 64, dtype=np.uint8)
    sb = rng.integers(118, 136, 64, dtype=np.uint8)
    d = _probe(2, a, b, sa, sb).view(np.float32).astype(np.float64)
    _check_f8(d, _f8_matrix(_e4m3_values(a), sa), _f8_matrix(_e4m3_values(b), sb), 2.0 ** -11)


def _f8_matrix32(lanes: np.ndarray, scales: np.ndarray | None = None, layout: str = "halves") -> np.ndarray:
    """The 32 x 64 operand the 32x32x64 f8f6f4 MFMA reads from 64 lanes x 32 bytes. "halves":
    lane group g = l/32 holds k in [16g, 16g+16) in bytes 0..15 and k in [32+16g, 48+16g) in bytes
    16..31; "runs": lane group g holds k in [32g, 32g+32). The E8M0 byte of row i's K block κ is
    lane i + 32κ's."""
    mat = np.zeros((32, 64))
    for lane in range(64):
        i, g = lane % 32, lane // 32
        if layout == "halves":
            mat[i, 16 * g:16 * g + 16] = lanes[lane, :16]
            mat[i, 32 + 16 * g:48 + 16 * g] = lanes[lane, 16:]
        else:
            mat[i, 32 * g:32 * g + 32] = lanes[lane]
    if scales is not None:
        for i in range(32):
            for kb in range(2):
                mat[i, 32 * kb:32 * kb + 32] *= 2.0 ** (float(scales[i + 32 * kb]) - 127)
    return mat


def _f8_32_error(d: np.ndarray, a: np.ndarray, b: np.ndarray) -> float:
    """Largest error of a 32x32 result (lane l, register r = row 8·(r/4) + 4·(l/32) + r%4 of
    column l%32) against the CPU product, relative to the sum of the products' magnitudes."""
    want, size = a @ b.T, np.abs(a) @ np.abs(b).T
    worst = 0.0
    for lane in range(64):
        for r in range(16):
            i, j = 8 * (r // 4) + 4 * (lane // 32) + r % 4, lane % 32
            worst = max(worst, abs(d[lane, r] - want[i, j]) / (size[i, j] + 1e-30))
    return worst


def test_mfma_f8_32x32_layout():
    """32x32x64 e4m3: the 32x32 output layout of the int8 32x32x32 form. (Unscaled, any K order
    common to both operands gives the same product; the scaled test below fixes the K order.)"""
    rng = np.random.default_rng(11)
    a, b = _e4m3_lanes(rng), _e4m3_lanes(rng)
    d = _probe(5, a, b).view(np.float32).astype(np.float64)
    err = _f8_32_error(d, _f8_matrix32(_e4m3_values(a)), _f8_matrix32(_e4m3_values(b)))
    assert err <= 2.0 ** -11, err


def test_mfma_f8_32x32_scaled_layout():
    """The K order ("halves": lane group g holds 16-byte chunks g and g+2 of a 64-byte K step)
    and the scale lanes (row (column) i, K block κ from lane i + 32κ) of the 32x32x64 form."""
    rng = np.random.default_rng(12)
    a, b = _e4m3_lanes(rng), _e4m3_lanes(rng)
    sa = rng.integers(118, 136, 64, dtype=np.uint8)
    sb = rng.integers(118, 136, 64, dtype=np.uint8)
    d = _probe(6, a, b, sa, sb).view(np.float32).astype(np.float64)
    va, vb = _e4m3_values(a), _e4m3_values(b)
    errs = {lay: _f8_32_error(d, _f8_matrix32(va, sa, lay), _f8_matrix32(vb, sb, lay))
            for lay in ("halves", "runs")}
    assert errs["halves"] <= 2.0 ** -11, errs


def test_mfma_bf16_layout():
    rng = np.random.default_rng(3)
    a = torch.randn(64, 16, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    b = torch.randn(64, 16, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    d = _probe(3, a.view(torch.uint8).numpy(), b.view(torch.uint8).numpy()).view(np.float32)
    want = _expand(a[:, :8].double().numpy(), 8) @ _expand(b[:, :8].double().numpy(), 8).T
    _check_layout(d.astype(np.float64), want, exact=False)
    del rng


def _out32(d: np.ndarray, want: np.ndarray) -> list[tuple[int, int, float, float]]:
    """(lane, register, got, want) wherever a 32x32 result misses `want` (register r of lane l
    holds row 8·(r/4) + 4·(l/32) + r%4 of column l%32)."""
    return [(lane, r, float(d[lane, r]), float(want[8 * (r // 4) + 4 * (lane // 32) + r % 4, lane % 32]))
            for lane in range(64) for r in range(16)
            if d[lane, r] != np.float32(want[8 * (r // 4) + 4 * (lane // 32) + r % 4, lane % 32])]  # fmt: skip


def test_mfma_f32_32x32x2_layout_and_exact_products():
    """32x32x2 f32: lane l supplies row (column) l%32 at K index l/32. Fed the svdq GEMM's offset
    operands (-1.5·2^23·sw with 12 significant bits, sa with 11), each product is exact in float32
    and the two-term sum is rounded once: every output equals float32 of the float64 sum."""
    rng = np.random.default_rng(7)
    sw = rng.uniform(0.004, 0.02, 64).astype(np.float16).astype(np.float64)
    sa = rng.uniform(0.3, 8.0, 64).astype(np.float16).astype(np.float64)
    a = np.zeros((64, 8), np.float32)
    b = np.zeros((64, 8), np.float32)
    a[:, 0] = -12582912.0 * sw
    b[:, 0] = sa
    assert np.array_equal(a[:, 0].astype(np.float64), -12582912.0 * sw)
    d = _probe(7, a, b).view(np.float32)
    mat_a = np.zeros((32, 2))
    mat_b = np.zeros((2, 32))
    for lane in range(64):
        mat_a[lane % 32, lane // 32] = a[lane, 0]
        mat_b[lane // 32, lane % 32] = b[lane, 0]
    misses = _out32(d, mat_a @ mat_b)
    assert not misses, (len(misses), misses[:4])


def test_mfma_f16_32x32x16_layout():
    """32x32x16 f16: lane l supplies row (column) l%32 and K slice 8·(l/32).. +8; every product
    of two fp16 values is exact in float32, so with one nonzero k the output is exact."""
    rng = np.random.default_rng(8)
    a = rng.uniform(-4, 4, (64, 16)).astype(np.float16)
    b = rng.uniform(-4, 4, (64, 16)).astype(np.float16)
    a[:, 8:] = 0
    b[:, 8:] = 0
    d = _probe(8, a, b).view(np.float32).astype(np.float64)
    mat_a = np.zeros((32, 16))
    mat_b = np.zeros((16, 32))
    for lane in range(64):
        mat_a[lane % 32, 8 * (lane // 32):8 * (lane // 32) + 8] = a[lane, :8]
        mat_b[8 * (lane // 32):8 * (lane // 32) + 8, lane % 32] = b[lane, :8]
    want = mat_a @ mat_b
    for lane in range(64):
        for r in range(16):
            ref = want[8 * (r // 4) + 4 * (lane // 32) + r % 4, lane % 32]
            assert abs(d[lane, r] - ref) <= 1e-6 * (1 + abs(ref)), (lane, r)
    one = np.zeros((64, 16), np.float16)
    other = np.zeros((64, 16), np.float16)
    one[:32, 0] = a[:32, 0]  # K = 1: lane group 0's element 0
    other[:32, 0] = b[:32, 0]
    d1 = _probe(8, one, other).view(np.float32)
    want1 = np.outer(one[:32, 0].astype(np.float64), other[:32, 0].astype(np.float64))
    assert not _out32(d1, want1)


# ------------------------------------------------------------------------ int8 lane

QUANT_SHAPES = [(1, 256), (3, 1024), (300, 3072), (64, 4352), (5, 32768), (257, 12288)]


@pytest.mark.parametrize("rotation", [256, 128, 0])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", QUANT_SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_int8_quantize_bit_exact(ops, rotation, dtype, shape):
    m, k = shape
    x = activations(m, k, seed=m * 7 + k, dtype=dtype)
    x[m // 2] = 0  # an all-zero row takes the scale floor
    if m > 2:
        x[1] *= 1e-6  # a tiny row
    if rotation == 256:
        q, s = ops.int8_quantize(x.to(DEV))
    else:
        q, s = ops.int8_quantize_rot(x.to(DEV), rotation)
    wq, ws = laws.quantize_rows_int8(x, rotation)
    assert torch.equal(q.cpu(), wq)
    assert torch.equal(s.cpu().view(torch.int32), ws.reshape(-1).view(torch.int32))


@pytest.mark.parametrize("rotation", [256, 128, 0])
@pytest.mark.parametrize("shape", [(4100, 2304), (3073, 4096), (6500, 768), (2, 1280)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_int8_row_quantize_strides_and_passes(ops, rotation, shape):
    """The one-wave-per-row quantizer (rows of at most 4096 elements): more rows than the grid
    has waves (each wave takes several rows, the next one's loads in flight), a second LDS pass
    that covers part of the row (2304 = 2048 + 256), rows that are not whole passes; codes and
    scales bit-exact, an all-zero row and a row of subnormal-scale values included."""
    m, k = shape
    if rotation == 128 and k % 128:
        pytest.skip("K is a multiple of the rotation")
    x = activations(m, k, seed=m + 3 * k)
    x[m - 1] = 0
    x[0] *= 1e-30
    q, s = ops.int8_quantize_rot(x.to(DEV), rotation)
    wq, ws = laws.quantize_rows_int8(x, rotation)
    assert torch.equal(q.cpu(), wq)
    assert torch.equal(s.cpu().view(torch.int32), ws.reshape(-1).view(torch.int32))


GEMM_SHAPES = [(1, 8, 256), (300, 512, 1024), (257, 264, 384), (64, 1032, 3072), (513, 256, 4096)]


@pytest.mark.parametrize("shape", GEMM_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_int8_accumulators_bit_exact(ops, shape):
    m, n, k = shape
    gen = torch.Generator().manual_seed(m + n + k)
    q = torch.randint(-127, 128, (m, k), generator=gen, dtype=torch.int8)
    w = torch.randint(-127, 128, (n, k), generator=gen, dtype=torch.int8)
    acc = ops.int8_acc(q.to(DEV), w.to(DEV))
    assert torch.equal(acc.cpu(), laws.int32_gemm(q, w))


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(3, 512, 1024), (300, 512, 1024), (257, 264, 768),
                                   (1, 1032, 4096), (16, 136, 256), (64, 520, 1024),
                                   (129, 264, 768), (256, 2048, 512), (4, 6144, 768),
                                   (3, 8192, 512), (4, 6136, 256)],
                         ids=lambda s: "x".join(map(str, s)))  # fmt: skip
def test_int8_linear_bit_exact(ops, shape, dtype, bias):
    """The whole int8.convrot linear (quantize + GEMM + epilogue) equals the CPU law bit for bit,
    with the probe's recipe (`internal/prebuilt.py:616-623`): random int8 data, scales ~1e-3.
    4 x 6144 and 3 x 8192 take quantize + GEMM by the few-row route rule, 4 x 6136 (just below
    it) the one-launch GEMV."""
    m, n, k = shape
    gen = torch.Generator().manual_seed(20261017 + m)
    data = torch.randint(-127, 128, (n, k), generator=gen, dtype=torch.int8)
    scale = (torch.randn(n, generator=gen).abs() + 0.5) * 1e-3
    b = torch.randn(n, generator=gen).to(dtype) if bias else None
    x = torch.randn(m, k, generator=gen).to(dtype)
    got = ops.int8_linear(x.to(DEV), data.to(DEV), scale.to(DEV),
                          None if b is None else b.to(DEV), dtype)  # fmt: skip
    want = laws.int8_linear(x, data, scale, b, dtype)
    assert torch.equal(got.cpu(), want)


GEMV_SHAPES = [(1, 256), (1, 768), (1, 3072), (1, 4096), (1, 8192), (1, 12288), (1, 16384),
               (1, 24576), (1, 32768), (2, 3072), (2, 8192), (2, 12288), (2, 16384), (3, 1024),
               (3, 4096), (3, 12288), (4, 2304), (4, 4096), (4, 8192), (4, 12288)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("shape", GEMV_SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_int8_gemv_bit_exact(ops, shape, dtype):
    """The fused few-row int8 linear (`cozyq_gemv`: rotation, per-row int8 and the GEMV in one
    launch) is served for M <= 4 up to K = 32768 (M = 1), 16384 (M = 2) and 12288 (M = 3, 4), the
    reference's range (`rotate.cu:453-468`) and more, and equals the CPU law bit for bit: codes from
    the rotation, exact int32 products, the epilogue's roundings. Rows include an all-zero row
    (the scale floor) and an outlier channel; N = 1032 leaves a ragged last workgroup."""
    from cozyq import _lib

    m, k = shape
    n = 1032
    gen = torch.Generator().manual_seed(20261210 + 7 * m + k)
    data = torch.randint(-127, 128, (n, k), generator=gen, dtype=torch.int8)
    scale = (torch.randn(n, generator=gen).abs() + 0.5) * 1e-3
    x = torch.randn(m, k, generator=gen)
    x[:, k // 3] *= 40
    if m > 1:
        x[1] = 0
    x = x.to(dtype)
    for b in (None, torch.randn(n, generator=gen).to(dtype)):
        out = torch.empty(m, n, dtype=dtype, device=DEV)
        xd, wd, sd = x.to(DEV), data.to(DEV), scale.to(DEV)
        bd = None if b is None else b.to(DEV)
        code = _lib.load().cozyq_gemv(0, xd.data_ptr(), int(dtype == torch.float16), wd.data_ptr(),
                                      sd.data_ptr(), None if bd is None else bd.data_ptr(),
                                      out.data_ptr(), int(dtype == torch.float16), m, n, k,
                                      torch.cuda.current_stream().cuda_stream)  # fmt: skip
        assert code == 0, _lib.error_name(code)
        assert torch.equal(out.cpu(), laws.int8_linear(x, data, scale, b, dtype))


@pytest.mark.parametrize("shape", [(2, 16640), (3, 12544), (4, 12544)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_int8_gemv_declines_wide_rows(ops, shape):
    """Past its widest rows (K > 16384 at M = 2, > 12288 at M = 3 and 4) the GEMV answers
    NOT_SUPPORTED and `int8_linear` quantizes + GEMMs, as the reference's caller does
    (`internal/prebuilt.py:99-118`): still bit-exact."""
    from cozyq import _lib

    lib = _lib.load()
    m, k = shape
    n = 264
    gen = torch.Generator().manual_seed(5 + k)
    data = torch.randint(-127, 128, (n, k), generator=gen, dtype=torch.int8)
    scale = (torch.randn(n, generator=gen).abs() + 0.5) * 1e-3
    x = torch.randn(m, k, generator=gen).to(torch.bfloat16)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    xd, wd, sd = x.to(DEV), data.to(DEV), scale.to(DEV)
    code = lib.cozyq_gemv(0, xd.data_ptr(), 0, wd.data_ptr(), sd.data_ptr(), None, out.data_ptr(),
                          0, m, n, k, torch.cuda.current_stream().cuda_stream)  # fmt: skip
    assert code == lib.cozyq_not_supported()
    got = ops.int8_linear(xd, wd, sd, None, torch.bfloat16)
    assert torch.equal(got.cpu(), laws.int8_linear(x, data, scale, None, torch.bfloat16))


@pytest.mark.parametrize("rotation", [0, 128, 256])
def test_int8_gemm_rotation_lanes_and_gelu(ops, rotation):
    m, n, k = 200, 264, 1024
    x = activations(m, k, seed=11)
    w = weights(n, k, seed=12)
    data, scale = laws.int8_weight_rotated(w, rotation) if rotation else laws.int8_weight_rowwise(w)
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(13)) * 0.1).to(torch.bfloat16)
    q, s = ops.int8_quantize_rot(x.to(DEV), rotation)
    plain = ops.int8_gemm_ex(q, s, data.to(DEV), scale.to(DEV), bias.to(DEV), torch.bfloat16, 0)
    assert torch.equal(plain.cpu(), laws.int8_linear(x, data, scale, bias, torch.bfloat16, rotation))
    gelu = ops.int8_gemm_ex(q, s, data.to(DEV), scale.to(DEV), bias.to(DEV), torch.bfloat16, 1)
    assert_close(gelu, laws.int8_exact(x, data, scale, bias, rotation, gelu=True))
    # and the rotated product approximates the unquantized linear
    ref = x.double() @ w.double().t() + bias.double()
    rel = (plain.cpu().double() - ref).norm() / ref.norm()
    assert rel < 0.05


@pytest.mark.parametrize("m", [3, 5, 20, 40, 100])
def test_int8_narrow_ragged_k_bit_exact(ops, m):
    """Few rows (the GEMV on the quantized rows at 3, the 16-row weight tile at 5 and 20, the
    narrow tiles beyond) with K = 1040, a last 128-byte step only partly inside the rows: the
    rotation-free lane, bit-exact to the CPU law."""
    n, k = 264, 1040
    x = activations(m, k, seed=71 + m)
    data, scale = laws.int8_weight_rowwise(weights(n, k, seed=72))
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(73)) * 0.1).to(torch.bfloat16)
    q, s = ops.int8_quantize_rot(x.to(DEV), 0)
    got = ops.int8_gemm_ex(q, s, data.to(DEV), scale.to(DEV), bias.to(DEV), torch.bfloat16, 0)
    assert torch.equal(got.cpu(), laws.int8_linear(x, data, scale, bias, torch.bfloat16, 0))


def test_int8_output_into_wider_rows(ops):
    """`out` with rows `ldo` apart (a sibling's column range of a packed output) is written in
    place (`internal/prebuilt.py:449-460`)."""
    m, n, k = 100, 256, 512
    x = activations(m, k, seed=21)
    data, scale = laws.int8_weight_rotated(weights(n, k, 22), 256)
    packed = torch.zeros(m, 3 * n, dtype=torch.bfloat16, device=DEV)
    view = packed[:, n:2 * n]
    q, s = ops.int8_quantize(x.to(DEV))
    got = ops.int8_gemm(q, s, data.to(DEV), scale.to(DEV), None, torch.bfloat16, out=view)
    assert got.data_ptr() == view.data_ptr()
    want = laws.int8_linear(x, data, scale, None, torch.bfloat16)
    assert torch.equal(packed[:, n:2 * n].cpu(), want)
    assert (packed[:, :n] == 0).all() and (packed[:, 2 * n:] == 0).all()


# (M, N, K): the GEMV's row counts on one batch of 1 KiB spans and on two (a partial last span),
# and at their widest K (32768 at M = 1, 16384 at 2, 12288 at 3..4); the row tile's 5..32 rows
# in one and two activation blocks, past its K (4352) and past its rows (33); N ragged against
# the workgroup's 16 rows.
CODES_GEMV_SHAPES = [(1, 264, 256), (2, 1032, 1280), (3, 136, 4352), (4, 264, 3072),
                     (4, 520, 12288), (3, 264, 12288), (2, 136, 16384), (1, 264, 32768),
                     (5, 136, 256), (8, 1032, 1280), (16, 264, 3072), (16, 136, 4352),
                     (17, 520, 4096), (24, 136, 1280), (32, 1032, 2048), (33, 264, 1024)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("shape", CODES_GEMV_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_int8_few_rows_gemm_bit_exact(ops, shape, dtype):
    """`cozyq_gemm`'s int8 product at few rows (config -1: the GEMV on the quantized rows at
    1..4, the 16-row weight tile at 5..32 with K <= 4096 and N <= 4096) equals the int8 law and
    the 128x64 tile bit for bit, with and without bias, and writes in place into rows `ldo`
    apart."""
    m, n, k = shape
    x = activations(m, k, seed=m * 11 + k)
    data, scale = laws.int8_weight_rowwise(weights(n, k, seed=n + k))
    b = (torch.randn(n, generator=torch.Generator().manual_seed(k)) * 0.1).to(dtype)
    q, s = ops.int8_quantize(x.to(DEV))
    for bias in (None, b):
        want = laws.int8_product(q.cpu(), s.cpu(), data, scale, dtype)
        want = want if bias is None else want + bias
        dev_bias = None if bias is None else bias.to(DEV)
        got = ops.int8_gemm(q, s, data.to(DEV), scale.to(DEV), dev_bias, dtype, -1)
        assert torch.equal(got.cpu(), want), bias is None
        assert torch.equal(got, ops.int8_gemm(q, s, data.to(DEV), scale.to(DEV), dev_bias, dtype, 2))
    packed = torch.zeros(m, 3 * n, dtype=dtype, device=DEV)
    ops.int8_gemm(q, s, data.to(DEV), scale.to(DEV), b.to(DEV), dtype, -1, out=packed[:, n:2 * n])
    assert torch.equal(packed[:, n:2 * n].cpu(), want)
    assert (packed[:, :n] == 0).all() and (packed[:, 2 * n:] == 0).all()


# ------------------------------------------------------------------------- fp8 lane


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(1, 16), (3, 1024), (300, 4096), (17, 4112), (4, 32768)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_fp8_quantize_bit_exact(ops, shape, dtype):
    m, k = shape
    x = activations(m, k, seed=m + k, dtype=dtype)
    x[0, :3] = torch.tensor([1e-7, -3e-5, 0.0]).to(dtype)  # subnormal e4m3 codes
    if m > 2:
        x[m - 1] = 0
    q, s = ops.fp8_quantize(x.to(DEV))
    wq, ws = laws.fp8_quantize(x)
    assert torch.equal(q.cpu().view(torch.uint8), wq.view(torch.uint8))
    assert torch.equal(s.cpu().view(torch.int32), ws.reshape(-1).view(torch.int32))


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("shape", [(300, 512, 1024), (257, 264, 4096), (64, 1024, 2064),
                                   (1, 8, 128), (16, 136, 4096), (33, 200, 1040), (100, 520, 1040),
                                   (129, 264, 4096), (256, 2048, 4096), (512, 1024, 4096),
                                   (1000, 776, 2064), (4096, 520, 4096)],
                         ids=lambda s: "x".join(map(str, s)))  # fmt: skip
def test_fp8_gemm_within_tolerance(ops, shape, bias):
    m, n, k = shape
    x = activations(m, k, seed=31 + m)
    data, scale = laws.fp8_weight(weights(n, k, seed=32))
    b = (torch.randn(n, generator=torch.Generator().manual_seed(33)) * 0.1).to(torch.bfloat16) \
        if bias else None
    q, s = ops.fp8_quantize(x.to(DEV))
    got = ops.fp8_gemm(q, s, data.to(DEV), scale.to(DEV), None if b is None else b.to(DEV),
                       torch.bfloat16)  # fmt: skip
    assert_close(got, laws.fp8_exact(x, data, scale, b))


# (M, N, K): one row; ragged rows and columns on every tile; the 256x256 tile's ragged edges;
# more rows than the narrow tiles' 128; a K with a partial 128-byte step for fp8.
CONFIG_SHAPES = [(1, 264, 1024), (100, 520, 768), (300, 1032, 2048), (513, 264, 256),
                 (1100, 776, 1024), (77, 136, 4096), (16, 1032, 4096), (29, 264, 2048)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("shape", CONFIG_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_every_gemm_config_bit_equal(ops, shape, dtype):
    """Every tile config of `cozyq_gemm` (0..5 and the shape rule's -1) gives the int8 law bit
    for bit, with and without bias (as the reference checks each explicit tile,
    `internal/bench/gemm.py:418-435`); the fp8 configs agree with one another bit for bit (each
    output's K sum runs in the same MFMA order) and sit within tolerance of the exact law; a
    config past the table is refused."""
    from cozyq import prebuilt

    m, n, k = shape
    configs = list(range(-1, prebuilt.GEMM_CONFIGS))
    x = activations(m, k, seed=m * 7 + k)
    data, scale = laws.int8_weight_rowwise(weights(n, k, seed=n))
    b = (torch.randn(n, generator=torch.Generator().manual_seed(n)) * 0.1).to(dtype)
    q, s = ops.int8_quantize(x.to(DEV))
    for bias in (None, b):
        want = laws.int8_product(q.cpu(), s.cpu(), data, scale, dtype)
        want = want if bias is None else want + bias
        for config in configs:
            got = ops.int8_gemm(q, s, data.to(DEV), scale.to(DEV),
                                None if bias is None else bias.to(DEV), dtype, config)  # fmt: skip
            assert torch.equal(got.cpu(), want), (config, bias is None)
    with pytest.raises(ValueError, match=f"config {prebuilt.GEMM_CONFIGS}"):
        ops.int8_gemm(q, s, data.to(DEV), scale.to(DEV), None, dtype, prebuilt.GEMM_CONFIGS)
    if k % 16 == 0:
        f8, f8s = laws.fp8_weight(weights(n, k, seed=n + 1))
        q8, s8 = ops.fp8_quantize(x.to(DEV))
        outs = [ops.fp8_gemm(q8, s8, f8.to(DEV), f8s.to(DEV), b.to(DEV), dtype, c) for c in configs]
        for config, out in zip(configs, outs):
            assert torch.equal(out, outs[1]), config
        assert_close(outs[0], laws.fp8_exact(x, f8, f8s, b))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_partial_last_round_runs_half_width_tiles_bit_equal(ops, dtype):
    """Config 0 on a grid whose last round is at most half full (M=4096, N=4352: 272 tiles of
    256x256 on 256 CUs) runs its full round on 256x256 tiles and the last 256 columns as a second
    launch of 256x128 tiles. int8's outputs equal the law bit for bit, with and without bias;
    fp8's equal the 128x128 config's bits (each output's K sum in the same MFMA order) and sit
    within tolerance of the exact law."""
    m, n, k = 4096, 4352, 512
    x = activations(m, k, seed=4352)
    data, scale = laws.int8_weight_rowwise(weights(n, k, seed=4353))
    b = (torch.randn(n, generator=torch.Generator().manual_seed(4354)) * 0.1).to(dtype)
    q, s = ops.int8_quantize(x.to(DEV))
    wd, sd, bd = data.to(DEV), scale.to(DEV), b.to(DEV)
    want = laws.int8_product(q.cpu(), s.cpu(), data, scale, dtype)
    assert torch.equal(ops.int8_gemm(q, s, wd, sd, None, dtype, 0).cpu(), want)
    got = ops.int8_gemm(q, s, wd, sd, bd, dtype, 0)
    assert torch.equal(got.cpu(), want + b)
    assert torch.equal(got, ops.int8_gemm(q, s, wd, sd, bd, dtype, 1))
    f8, f8s = laws.fp8_weight(weights(n, k, seed=4355))
    q8, s8 = ops.fp8_quantize(x.to(DEV))
    outs = [ops.fp8_gemm(q8, s8, f8.to(DEV), f8s.to(DEV), bd, dtype, c) for c in (0, 1)]
    assert torch.equal(outs[0], outs[1])
    assert_close(outs[0], laws.fp8_exact(x, f8, f8s, b))


@pytest.mark.parametrize("shape", [(16, 520, 4112), (3, 264, 80), (32, 136, 1040)],
                         ids=lambda s: "x".join(map(str, s)))  # fmt: skip
def test_fp8_configs_partial_k_steps(ops, shape):
    """Where K ends inside a 128-byte step: every config gives the same bits (zeros past K, the
    same MFMA order), with bias, within tolerance of the exact law."""
    from cozyq import prebuilt

    m, n, k = shape
    x = activations(m, k, seed=m + k)
    f8, f8s = laws.fp8_weight(weights(n, k, seed=n + 3))
    b = (torch.randn(n, generator=torch.Generator().manual_seed(n)) * 0.1).to(torch.bfloat16)
    q8, s8 = ops.fp8_quantize(x.to(DEV))
    outs = [ops.fp8_gemm(q8, s8, f8.to(DEV), f8s.to(DEV), b.to(DEV), torch.bfloat16, c)
            for c in range(prebuilt.GEMM_CONFIGS)]  # fmt: skip
    for config, out in enumerate(outs):
        assert torch.equal(out, outs[1]), config
    assert_close(outs[4], laws.fp8_exact(x, f8, f8s, b))


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(300, 512, 1024), (520, 264, 2064), (40, 136, 4096)],
                         ids=lambda s: "x".join(map(str, s)))  # fmt: skip
def test_fp8_gemm_gelu_and_fp16_within_tolerance(ops, shape, out_dtype):
    """The fp8 GEMM's tanh-GELU epilogue through the C ABI (cozyq_gemm_ex, fp8 = 1): the law's
    rounded output (bias in float32), then GELU in float32 and one more rounding."""
    from cozyq import _lib

    m, n, k = shape
    x = activations(m, k, seed=35 + m)
    data, scale = laws.fp8_weight(weights(n, k, seed=36))
    b = (torch.randn(n, generator=torch.Generator().manual_seed(37)) * 0.1).to(torch.bfloat16)
    q, s = ops.fp8_quantize(x.to(DEV))
    out = torch.empty(m, n, dtype=out_dtype, device=DEV)
    bias = b.to(out_dtype).to(DEV)
    wd, ws = data.to(DEV), scale.to(DEV)
    code = _lib.load().cozyq_gemm_ex(0, 1, q.data_ptr(), s.data_ptr(), wd.data_ptr(), ws.data_ptr(),
                                     bias.data_ptr(), out.data_ptr(), n,
                                     int(out_dtype == torch.float16), m, n, k, 1,
                                     torch.cuda.current_stream().cuda_stream)  # fmt: skip
    assert code == 0
    rounded = laws.fp8_exact(x, data, scale, b.to(out_dtype)).to(out_dtype)
    assert_close(out, laws.gelu_tanh(rounded.float()).double())


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 13, 16])
@pytest.mark.parametrize("k", [4096, 1040, 16384, 8208])
def test_fp8_small_linear_within_tolerance(ops, m, k):
    n = 1032
    x = activations(m, k, seed=41 + m)
    data, scale = laws.fp8_weight(weights(n, k, seed=42))
    b = (torch.randn(n, generator=torch.Generator().manual_seed(43)) * 0.1).to(torch.bfloat16)
    got = ops.fp8_linear(x.to(DEV), data.to(DEV), scale.to(DEV), b.to(DEV), torch.bfloat16)
    assert got.shape == (m, n)
    assert_close(got, laws.fp8_exact(x, data, scale, b))


#: (M, N, K) through the fused fp8 kernels: the GEMV (M <= 4) and the row-tile kernel (5..16
#: rows, K <= 4096, and 3..4 rows of a wide weight: 4 x 14336, 3 x 12288), whose workgroups own
#: 8..64 weight rows (N = 14336: 56 rows, three whole 16-row tiles and a half; N = 2056: one
#: workgroup of 16 rows among 8-row ones; N = 16392: more 8-row units than 8 a CU, so more
#: workgroups than CUs) and whose waves split K (K = 16 and 400: waves with no K step or a
#: partial one).
FUSED_FP8_SHAPES = [(1, 14336, 4096), (3, 2056, 1040), (5, 14336, 4096), (9, 2056, 1040),
                    (16, 14336, 4096), (16, 16392, 1024), (12, 264, 16), (7, 520, 400),
                    (16, 8, 4096), (4, 14336, 4096), (3, 12288, 3072)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("shape", FUSED_FP8_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_fp8_fused_codes_bit_exact(ops, shape, dtype):
    """A selector weight (row n holds e4m3 1.0 at column n % K, scale 1) makes output n of row m
    the activation's code q[m][n % K] times the row's scale: one float32 product rounded to the
    output dtype, with no sum. So every code and scale the fused kernel made inside itself is
    held bit for bit against the law's (a zero's sign aside), at every K position each wave and
    lane group owns, and every output lands at its row and column."""
    from cozyq import prebuilt

    m, n, k = shape
    x = activations(m, k, seed=900 + m + k, dtype=dtype)
    x[0, :3] = torch.tensor([1e-7, -3e-5, 0.0]).to(dtype)  # subnormal codes and a zero
    if m > 2:
        x[m - 1] = 0  # a zero row: the scale floor
    data = torch.zeros(n, k, dtype=torch.uint8)
    data[torch.arange(n), torch.arange(n) % k] = 0x38  # e4m3 1.0
    data = data.view(torch.float8_e4m3fn)
    ones = torch.ones(n)
    got = ops.fp8_linear(x.to(DEV), data.to(DEV), ones.to(DEV), None, dtype)
    assert m <= prebuilt.FP8_SMALL_ROWS
    wq, ws = laws.fp8_quantize(x)
    picked = wq.float()[:, torch.arange(n) % k]
    assert torch.equal(got.cpu(), (picked * ws.reshape(-1, 1)).to(dtype))


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("dtypes", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.bfloat16),
                                    (torch.bfloat16, torch.float16)],
                         ids=["bf16", "fp16-in", "fp16-out"])  # fmt: skip
@pytest.mark.parametrize("shape", FUSED_FP8_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_fp8_fused_within_tolerance(ops, shape, dtypes, bias):
    """The fused fp8 kernels' sums (the row-tile kernel adds its waves' K slices in wave order)
    within tolerance of the float64 product of the law's codes, each input and output dtype,
    with and without bias; the same shape through quantize + GEMM agrees as closely."""
    m, n, k = shape
    x_dtype, out_dtype = dtypes
    x = activations(m, k, seed=950 + m + k, dtype=x_dtype)
    data, scale = laws.fp8_weight(weights(n, k, seed=951 + n))
    b = (torch.randn(n, generator=torch.Generator().manual_seed(952)) * 0.1).to(out_dtype) \
        if bias else None
    xd, wd, sd = x.to(DEV), data.to(DEV), scale.to(DEV)
    bd = None if b is None else b.to(DEV)
    got = ops.fp8_linear(xd, wd, sd, bd, out_dtype)
    exact = laws.fp8_exact(x, data, scale, b)
    assert_close(got, exact)
    q, s = ops.fp8_quantize(xd)
    assert_close(ops.fp8_gemm(q, s, wd, sd, bd, out_dtype), exact)


# ------------------------------------------------------------------ producer prologue

#: (name, norm, eps, tables, activation, up): the prologue shapes `int8_rows` forwards.
PROLOGUES = [
    ("rms", laws.NORM_RMS, 1e-6, False, 0, False),
    ("layer+gelu_tanh", laws.NORM_LAYER, 1e-5, False, laws.ACT_GELU_TANH, False),
    ("rms+tables+gelu", laws.NORM_RMS, 1e-6, True, laws.ACT_GELU, False),
    ("tables", 0, 0.0, True, 0, False),
    ("situ", 0, 0.0, False, laws.ACT_SITU, False),
    ("swiglu_up", 0, 0.0, False, laws.ACT_SWIGLU, True),
    ("swiglu_halves", 0, 0.0, False, laws.ACT_SWIGLU, False),
]


@pytest.mark.parametrize("fp8", [False, True], ids=["int8", "fp8"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("case", PROLOGUES, ids=[c[0] for c in PROLOGUES])
def test_quantize_prologue_within_one_step(ops, fp8, dtype, case):
    """The producer prologue folded into the quantize pass, against the CPU law on the same
    rows. Its norm sums and transcendentals are the platform's, not torch CPU's, so the check is
    a bound: scales within 1e-5 relative, every dequantized value within one quantization step
    (int8) or one e4m3 step (fp8), and at most 1% of codes different. SwiGLU rounds silu to the
    rows' dtype, where a one-ulp float32 difference can move a bf16 value by a whole step (and
    with the row maximum, the scale): its bounds are 2^-7, two steps and 5%."""
    name, norm, eps, tables, act, with_up = case
    m, k = (48, 4112) if fp8 else (48, 3072)
    gated = act == laws.ACT_SITU or (act == laws.ACT_SWIGLU and not with_up)
    x = activations(m, 2 * k if gated else k, seed=500 + PROLOGUES.index(case), dtype=dtype)
    gen = torch.Generator().manual_seed(71)
    scale = shift = up = None
    if tables:  # two table rows over the 48 rows: rows_per_entry 24
        scale = (torch.randn(2, k, generator=gen) * 0.2).to(dtype)
        shift = (torch.randn(2, k, generator=gen) * 0.2).to(dtype)
    if with_up:
        up = activations(m, k, seed=72, dtype=dtype)
    dev = lambda t: None if t is None else t.to(DEV)  # noqa: E731
    quantize = ops.fp8_quantize if fp8 else ops.int8_quantize
    q, s = quantize(x.to(DEV), dev(scale), dev(shift), norm, eps, act, dev(up))
    rows = laws.prologue(x, scale=scale, shift=shift, norm=norm, eps=eps, activation=act, up=up)
    if fp8:
        wq, ws = laws.fp8_quantize(rows)
        got, want = q.cpu().float(), wq.float()
        step = (want.abs() * 2.0**-3).clamp(min=2.0**-9)  # one e4m3 step at the value
    else:
        wq, ws = laws.quantize_rows_int8(rows, 256)
        got, want = q.cpu().float(), wq.float()
        step = torch.ones_like(want)
    s, ws = s.cpu().reshape(-1, 1), ws.reshape(-1, 1)
    swiglu = act == laws.ACT_SWIGLU
    assert ((s - ws).abs() <= (2.0**-7 if swiglu else 1e-5) * ws).all()
    assert ((got * s - want * ws).abs() <= (2.01 if swiglu else 1.01) * step * ws + 1e-30).all()
    assert (got != want).float().mean() <= (0.05 if swiglu else 0.01)


# ------------------------------------------------------------------------- w4a8 lane


def _w4a8(n: int, k: int, seed: int, codebook: bool):
    """A w4a8.convrot weight with the probe's recipe (`internal/prebuilt.py:695-706`): random
    code bytes, E4M3 group scales |N(0,1)|·40 + 16 clamped to 440, row scales ~1e-3."""
    from cozyq import prebuilt

    gen = torch.Generator().manual_seed(seed)
    codes = torch.randint(0, 256, (n, k // 2), generator=gen, dtype=torch.uint8)
    gs = (torch.randn(n, k // 16, generator=gen).abs() * 40 + 16).clamp(max=440).to(torch.float8_e4m3fn)
    scale = (torch.randn(n, generator=gen).abs() + 0.5) * 1e-3
    book = torch.tensor(laws.W4A8_CODEBOOK) if codebook else None
    dev = prebuilt.W4a8(codes.to(DEV), gs.to(DEV), scale.to(DEV), None if book is None else book.to(DEV))
    return dev, laws.w4a8_unpack(codes, gs, book), scale


@pytest.mark.parametrize("codebook", [True, False], ids=["codebook", "uniform"])
def test_w4a8_unpack_every_scale_byte_bit_exact(ops, codebook):
    """`cozyq_w4a8_unpack` over a weight whose 256 rows carry the 256 E4M3 scale bytes (NaN
    included) and random codes: every level equals the CPU law."""
    from cozyq import prebuilt

    gen = torch.Generator().manual_seed(9)
    codes = torch.randint(0, 256, (256, 512), generator=gen, dtype=torch.uint8)
    gs = torch.arange(256, dtype=torch.uint8).reshape(256, 1).expand(256, 64).contiguous()
    gs = gs.view(torch.float8_e4m3fn)
    book = torch.tensor(laws.W4A8_CODEBOOK) if codebook else None
    w = prebuilt.W4a8(codes.to(DEV), gs.to(DEV), torch.ones(256, device=DEV),
                      None if book is None else book.to(DEV))  # fmt: skip
    assert torch.equal(ops.w4a8_unpack(w).cpu(), laws.w4a8_unpack(codes, gs, book))


@pytest.mark.parametrize("codebook", [True, False], ids=["codebook", "uniform"])
@pytest.mark.parametrize("shape", [(1, 264, 1024), (3, 520, 1024), (2, 12288, 3072), (4, 12288, 3072), (4, 1032, 8192),
                                   (1, 136, 256), (16, 136, 256), (5, 520, 1024), (9, 1032, 8192),
                                   (13, 264, 768), (16, 12288, 3072), (100, 256, 3072), (256, 512, 768),
                                   (300, 520, 1024), (17, 136, 4096), (24, 520, 1024), (32, 1032, 3072),
                                   (32, 264, 4096)],
                         ids=lambda s: "x".join(map(str, s)))  # fmt: skip
def test_w4a8_linear_bit_exact(ops, shape, codebook):
    """The w4a8 linear (int8.convrot's operand; the GEMV form at 1..2 rows, the row-tile kernel
    at 3..16 and, in two activation blocks, at 17..32 rows with M·K ≤ 98304 and K ≤ 4096, the
    fused unpack-in-registers GEMM up to 256 rows, unpack + the int8 GEMM beyond)
    equals the int8 CPU law on the unpacked levels, bit for bit, with and without bias; the
    fused and unpack configs agree bit for bit."""
    from cozyq import prebuilt

    m, n, k = shape
    w, levels, scale = _w4a8(n, k, 20261022 + m, codebook)
    gen = torch.Generator().manual_seed(m + k)
    x = torch.randn(m, k, generator=gen).to(torch.bfloat16)
    b = torch.randn(n, generator=gen).to(torch.bfloat16)
    for bias in (None, b):
        got = ops.w4a8_linear(x.to(DEV), w, None if bias is None else bias.to(DEV), torch.bfloat16)
        assert torch.equal(got.cpu(), laws.int8_linear(x, levels, scale, bias, torch.bfloat16))
    q, s = ops.int8_quantize(x.to(DEV))
    unpacked = ops.w4a8_gemm(q, s, w, b.to(DEV), torch.bfloat16, prebuilt.UNPACK)
    for config in range(1, prebuilt.GEMM_CONFIGS):  # every fused tile
        assert torch.equal(ops.w4a8_gemm(q, s, w, b.to(DEV), torch.bfloat16, config), unpacked), config


# ------------------------------------------------------------------------ MXFP8 lane


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(1, 32), (3, 1024), (300, 3072), (64, 12288)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_mx_quantize_bit_exact(ops, shape, dtype):
    m, k = shape
    x = activations(m, k, seed=51 + k, dtype=dtype)
    x = x * torch.logspace(-8, 8, m).reshape(-1, 1).to(dtype)
    x[0, :32] = 0  # a zero block
    q, s = ops.mx_quantize(x.to(DEV))
    wq, ws = laws.mx_quantize(x)
    assert torch.equal(q.cpu().view(torch.uint8), wq.view(torch.uint8))
    assert torch.equal(s.cpu(), ws)


@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("shape", [(300, 512, 1024), (257, 264, 3072), (1, 8, 128),
                                   (512, 1024, 4096), (260, 264, 12288)],
                         ids=lambda s: "x".join(map(str, s)))  # fmt: skip
def test_mx_gemm_within_tolerance(ops, shape, bias):
    m, n, k = shape
    x = activations(m, k, seed=61 + m)
    data, wbyte = laws.mx_quantize(weights(n, k, seed=62))
    b = (torch.randn(n, generator=torch.Generator().manual_seed(63)) * 0.1).to(torch.bfloat16) \
        if bias else None
    q, qs = ops.mx_quantize(x.to(DEV))
    got = ops.mx_gemm(q, qs, data.to(DEV), wbyte.to(DEV), None if b is None else b.to(DEV),
                      torch.bfloat16)  # fmt: skip
    assert_close(got, laws.mx_exact(x, data, wbyte, b))


# ------------------------------------------------------------------ full-size property


def test_c1_full_size_rowwise_int8_bit_exact(ops):
    """BASELINE config 1 at its real shape (M=128, K=N=3072): no rotation, per-token int8
    activations and the per-output-channel int8 weight law (`internal/probe.py:764-767`).
    Codes, scales, int32 accumulators and the bf16 output, without and with a bias, all equal
    the CPU law bit for bit."""
    m, k, n = 128, 3072, 3072
    x = activations(m, k, seed=20261201)
    data, scale = laws.int8_weight_rowwise(weights(n, k, seed=20261211))
    q, s = ops.int8_quantize_rot(x.to(DEV), 0)
    wq, ws = laws.quantize_rows_int8(x, 0)
    assert torch.equal(q.cpu(), wq)
    assert torch.equal(s.cpu().view(torch.int32), ws.reshape(-1).view(torch.int32))
    wd, sd = data.to(DEV), scale.to(DEV)
    assert torch.equal(ops.int8_acc(q, wd).cpu(), laws.int32_gemm(wq, data))
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(12)) * 0.1).to(torch.bfloat16)
    for b in (None, bias):
        got = ops.int8_gemm_ex(q, s, wd, sd, None if b is None else b.to(DEV), torch.bfloat16, 0)
        assert torch.equal(got.cpu(), laws.int8_linear(x, data, scale, b, torch.bfloat16, rotation=0))


@pytest.fixture(scope="module")
def c3_weight():
    """Config 3's fp8 weight (N=14336, K=4096) by the per-row E4M3 law, shared by the M sweep."""
    data, scale = laws.fp8_weight(weights(14336, 4096, seed=20261204))
    return data, scale


@pytest.mark.parametrize("m", [1, 16, 256])
def test_c3_decode_shapes_within_tolerance(ops, c3_weight, m):
    """BASELINE config 3 at M = 1, 16 and 256 on its real weight (K=4096, N=14336), through the
    leaf's own route (`fp8_linear`: the fused quantize + GEMV for M <= 4, quantize + the narrow
    GEMM above): every output row within tolerance of the float64 product of the law's codes,
    and for M > 4 the activation's codes and scales bit-exact."""
    data, scale = c3_weight
    k, n = 4096, 14336
    x = activations(m, k, seed=20261203 + m)
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(7)) * 0.1).to(torch.bfloat16)
    wd, sd, bd = data.to(DEV), scale.to(DEV), bias.to(DEV)
    got = ops.fp8_linear(x.to(DEV), wd, sd, bd, torch.bfloat16)
    assert got.shape == (m, n)
    assert_close(got, laws.fp8_exact(x, data, scale, bias))
    if m > 4:
        q, s = ops.fp8_quantize(x.to(DEV))
        wq, ws = laws.fp8_quantize(x)
        assert torch.equal(q.cpu().view(torch.uint8), wq.view(torch.uint8))
        assert torch.equal(s.cpu().view(torch.int32), ws.reshape(-1).view(torch.int32))



def test_c3_full_size_fp8_codes_and_sampled_rows(ops):
    """BASELINE config 3 at M=4096 (K=4096, N=14336): every e4m3 code and scale of the
    activation bit-exact, and 2 rows of every M-tile (32, each against every column) within
    tolerance of the float64 product; the whole output finite."""
    m, k, n = 4096, 4096, 14336
    x = activations(m, k, seed=20261203)
    data, scale = laws.fp8_weight(weights(n, k, seed=20261204))
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(7)) * 0.1).to(torch.bfloat16)
    q, s = ops.fp8_quantize(x.to(DEV))
    wq, ws = laws.fp8_quantize(x)
    assert torch.equal(q.cpu().view(torch.uint8), wq.view(torch.uint8))
    assert torch.equal(s.cpu().view(torch.int32), ws.reshape(-1).view(torch.int32))
    out = ops.fp8_gemm(q, s, data.to(DEV), scale.to(DEV), bias.to(DEV), torch.bfloat16)
    rows = tile_rows(m, 2)
    exact = (wq[rows].double() @ data.double().t()) * ws[rows].double() * scale.double().reshape(1, -1)
    assert_close(out.cpu()[rows], exact + bias.double())
    assert math.isfinite(out.float().abs().max().item())


@pytest.mark.parametrize("shape", [(3072, 9216), (3072, 3072), (3072, 12288), (12288, 3072)],
                         ids=["qkv", "attn_out", "ffn_up", "ffn_down"])
def test_c5_full_size_mx_codes_and_sampled_rows(ops, shape):
    """BASELINE config 5 at M=4096 over the DiT block's four shapes: every e4m3 code and E8M0
    byte of the activation bit-exact, and 2 rows of every M-tile (32, each against every column)
    within tolerance of the float64 product of the dequantized operands."""
    k, n = shape
    m = 4096
    x = activations(m, k, seed=20261205 + k)
    data, wbyte = laws.mx_quantize(weights(n, k, seed=20261206 + n))
    q, qs = ops.mx_quantize(x.to(DEV))
    wq, wqs = laws.mx_quantize(x)
    assert torch.equal(q.cpu().view(torch.uint8), wq.view(torch.uint8))
    assert torch.equal(qs.cpu(), wqs)
    out = ops.mx_gemm(q, qs, data.to(DEV), wbyte.to(DEV), None, torch.bfloat16)
    rows = tile_rows(m, 2)
    exact = laws.mx_dequantize(wq[rows], wqs[rows]).double() @ laws.mx_dequantize(data, wbyte).double().t()
    assert_close(out.cpu()[rows], exact)
    assert math.isfinite(out.float().abs().max().item())


def test_c2_full_size_codes_and_sampled_rows(ops):
    """BASELINE config 2 at its real shape: every code and scale bit-exact; the whole int32
    accumulator matrix exact by its row and column checksums (weighted and plain, int64), and 4
    rows of every M-tile exactly; the bias + GELU outputs of those 64 rows, against every column,
    within tolerance of the float64 law; the whole output finite."""
    m, k, n = 4096, 3072, 12288
    x = activations(m, k, seed=20261202)
    w = weights(n, k, seed=20261203)
    data, scale = laws.int8_weight_rotated(w, 128)
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(5)) * 0.1).to(torch.bfloat16)
    q, s = ops.int8_quantize_rot(x.to(DEV), 128)
    wq, ws = laws.quantize_rows_int8(x, 128)
    assert torch.equal(q.cpu(), wq)
    assert torch.equal(s.cpu().view(torch.int32), ws.reshape(-1).view(torch.int32))
    out = ops.int8_gemm_ex(q, s, data.to(DEV), scale.to(DEV), bias.to(DEV), torch.bfloat16, 1)
    acc = ops.int8_acc(q, data.to(DEV)).cpu()
    checksums_exact(acc, wq, data, seed=6)
    rows = tile_rows(m)
    assert len(rows) == 64
    assert torch.equal(acc[rows], laws.int32_gemm(wq[rows], data))
    exact = laws.int32_gemm(wq[rows], data).double() * ws[rows].double() * scale.double()
    exact = laws.gelu_tanh((exact + bias.double()).float()).double()
    assert_close(out.cpu()[rows], exact)
    assert math.isfinite(out.float().abs().max().item())

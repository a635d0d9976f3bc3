"""GPU parity of the svdq.nvfp4 W4A4 lane (`cozyq_svdq_input_scale`, `cozyq_svdq_quantize`,
`cozyq_svdq_gemm`) against the CPU law (`oracle/laws.py`, restating
`internal/svdq_linear.py:582-659`).

Bar (the reference's own probe, `internal/svdq_linear.py:406-440`): g_x, the E2M1 codes and the
E4M3 scales bit-exact; la = bf16(x·downᵀ) within one bf16 rounding of its float64 product; the
output within |got − exact| ≤ ATOL·rms(exact) + RTOL·|exact| of the float64 law
(`laws.svdq_nvfp4_exact`), and bit-exact where every product and partial sum is exact in float32.
"""

from __future__ import annotations

import pytest
import torch

from oracle import laws

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
ATOL, RTOL = 1e-2, 2e-2


@pytest.fixture(scope="module")
def ops():
    from cozyq import prebuilt

    return prebuilt.library(0)


def assert_close(got: torch.Tensor, exact: torch.Tensor) -> None:
    got, exact = got.double().cpu(), exact.double().cpu()
    rms = exact.pow(2).mean().sqrt().item()
    err = (got - exact).abs()
    worst = (err - (ATOL * rms + RTOL * exact.abs())).max().item()
    assert worst <= 0, f"max excess {worst:.3g} (rms {rms:.3g}, max err {err.max().item():.3g})"


def activations(m: int, k: int, seed: int, dtype=torch.bfloat16) -> torch.Tensor:
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=gen)
    x[:, torch.randperm(k, generator=gen)[: max(1, k // 100)]] *= 20
    return x.to(dtype)


def roles(n: int, k: int, r: int, seed: int, channel: bool = True, stored: bool = False) -> dict:
    """A random svdq.nvfp4 leaf as the reference's probe draws one
    (`internal/svdq_linear.py:406-418`)."""
    gen = torch.Generator().manual_seed(seed)
    out = {
        "weight": torch.randint(0, 256, (n, k // 2), generator=gen).to(torch.uint8),
        "scale": (torch.randn(n, k // 16, generator=gen).abs() + 0.5).to(torch.float8_e4m3fn),
        "scale_2": torch.full((1,), 0.01),
        "pre_quant_scale": torch.randn(k, generator=gen).abs() + 0.5,
        "lowrank_down": (torch.randn(r, k, generator=gen) * 0.05).to(torch.bfloat16),
        "lowrank_up": (torch.randn(n, r, generator=gen) * 0.05).to(torch.bfloat16),
    }
    if channel:
        out["channel_scale"] = torch.randn(n, generator=gen).abs() + 0.5
    if stored:
        out["input_scale"] = torch.tensor([0.05])
    return out


def on(d: dict) -> dict:
    return {key: t.to(DEV) for key, t in d.items()}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("shape", [(1, 64), (300, 3072), (2, 4160), (4096, 3072)],
                         ids=lambda s: "x".join(map(str, s)))  # fmt: skip
def test_svdq_input_scale_bit_exact(ops, shape, dtype):
    m, k = shape
    x = activations(m, k, seed=m + k, dtype=dtype)
    p = torch.randn(k, generator=torch.Generator().manual_seed(k)).abs() + 0.5
    got = ops.svdq_input_scale(x.to(DEV), p.to(DEV))
    want = laws.svdq_nvfp4_input_scale(x, p)
    assert torch.equal(got.cpu().view(torch.int32), want.view(torch.int32))
    zero = ops.svdq_input_scale(torch.zeros(m, k, dtype=dtype, device=DEV), p.to(DEV))
    assert zero.item() == torch.tensor(1e-30).item()  # the law's floor


@pytest.mark.parametrize("rank", [32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("shape", [(1, 64), (17, 128), (300, 1024), (257, 3072), (2, 12352)],
                         ids=lambda s: "x".join(map(str, s)))  # fmt: skip
def test_svdq_quantize_bit_exact(ops, shape, dtype, rank):
    """Codes and scales bit for bit (every row's blocks, the scale floor of an all-zero row, the
    sign of -0), rows past M zero, la within one bf16 rounding of its float64 product."""
    m, k = shape
    x = activations(m, k, seed=3 * m + k, dtype=dtype)
    x[m // 2] = 0
    if m > 2:
        x[1, :16] = -0.0
    d = roles(264, k, rank, seed=k)
    g = laws.svdq_nvfp4_input_scale(x, d["pre_quant_scale"])
    act, ascales, la = ops.svdq_quantize(x.to(DEV), d["pre_quant_scale"].to(DEV), g.to(DEV),
                                         d["lowrank_down"].to(DEV))  # fmt: skip
    padded = -(-m // 256) * 256
    assert act.shape == (padded, k // 2) and ascales.shape == (padded, k // 16) and la.shape == (padded, rank)
    codes, scales = laws.svdq_nvfp4_quantize(laws.svdq_smooth(x, d["pre_quant_scale"]), g)
    assert torch.equal(act[:m].cpu(), laws.svdq_nvfp4_pack(codes))
    assert torch.equal(ascales[:m].cpu().view(torch.uint8), scales.view(torch.uint8))
    assert not act[m:].any() and not ascales[m:].view(torch.uint8).any() and not la[m:].view(torch.int16).any()
    # One bf16 rounding of the float64 product, plus float32 accumulation over K (2^-18 of the
    # sum of |terms|: where the terms cancel, float32 itself is off by more than a bf16 step).
    down = d["lowrank_down"].to(dtype).double()
    exact = x.double() @ down.t()
    spread = x.double().abs() @ down.abs().t()
    err = (la[:m].cpu().double() - exact).abs()
    assert (err <= exact.abs() * 2.0**-8 + spread * 2.0**-18).all(), err.max()


def test_e2m1_conversion_matches_the_threshold_law():
    """The quantizer's code conversion (`cozyq_probe_e2m1`: v_cvt_scalef32_pk_fp4_f32 at unit
    scale after its −0 and NaN fix-ups) against the law's threshold count
    (`laws.SVDQ_THRESHOLDS`, internal/svdq_linear.py:612-616; sign from xs < 0) on every float32
    of both signs in [2^-4, 2^4) (every threshold and the saturation past 6), and on zeros,
    subnormals, tiny and huge values, ±inf and NaN."""
    import numpy as np

    from cozyq import _lib

    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream

    def law(v: np.ndarray) -> np.ndarray:
        a = np.abs(v)
        code = np.zeros(v.shape, dtype=np.uint8)
        for bound, inclusive in laws.SVDQ_THRESHOLDS:
            code += (a >= bound) if inclusive else (a > bound)
        return code + (v < 0).astype(np.uint8) * 8

    def check(v: np.ndarray) -> None:
        tin = torch.from_numpy(v).to(DEV)
        tout = torch.empty(v.size // 2, dtype=torch.uint8, device=DEV)
        assert lib.cozyq_probe_e2m1(0, tin.data_ptr(), tout.data_ptr(), v.size, stream) == 0
        packed = tout.cpu().numpy()
        got = np.stack([packed & 0x0F, packed >> 4], axis=-1).reshape(-1)
        want = law(v)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, f"{bad.size} differ, e.g. {v[bad[:4]]} -> {got[bad[:4]]} vs {want[bad[:4]]}"

    for e in range(-4, 4):  # one binade [2^e, 2^(e+1)) of both signs at a time
        bits = (np.arange(1 << 23, dtype=np.uint32) | np.uint32((127 + e) << 23))
        v = bits.view(np.float32)
        check(np.concatenate([v, -v]))
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -np.nan, 1e-45, -1e-45, 1e-40, -1e-40,
                        1.1754944e-38, -1.1754944e-38, 1e-30, -1e-30, 0.1, -0.1, 16.0, -16.0, 1e30,
                        -1e30, 3.4028235e38, -3.4028235e38], dtype=np.float32)
    with np.errstate(invalid="ignore"):
        check(special)


def test_svdq_quantize_rounding_ties_bit_exact(ops):
    """Codes exactly at every rounding threshold of the law and one bf16 step either side
    (xs / (scale·g) = 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5; both signs), past the largest level
    (6.5, 7), at ±0, at subnormal and tiny xs: ties go to the even code, −0 codes as +0, a tiny
    negative as −0. g = 1 (the tensor's largest |x·p| is 2688) and, where a block holds 6, its
    scale is 1, so the quotients are the values themselves."""
    k, m = 256, 8
    thresholds = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]

    def bf(v: float) -> torch.Tensor:
        return torch.tensor(v, dtype=torch.bfloat16)

    def nudge(v: float, d: int) -> torch.Tensor:  # d bf16 steps away from v
        return (bf(v).view(torch.int16) + d).view(torch.bfloat16)

    blocks = [torch.stack([bf(6.0), bf(t), nudge(t, 1), nudge(t, -1), -bf(t), -nudge(t, 1), -nudge(t, -1)]
                          + [bf(0.0)] * 9) for t in thresholds]  # fmt: skip
    x = torch.zeros(m, k, dtype=torch.bfloat16)
    for r in range(m):
        for b, blk in enumerate(blocks):
            at = 16 * ((b + r) % 16)
            x[r, at:at + 16] = blk
    x[0, 255] = 2688.0
    x[1, 200:204] = torch.tensor([-0.0, 0.0, 1e-40, -1e-40]).to(torch.bfloat16)
    x[2, 200:216] = torch.tensor([7.0, 6.5, -7.0, 1e-3, -1e-3, 0.0, -0.0, 3.0] * 2).to(torch.bfloat16)
    x[4, 232:248] = torch.tensor([1e-30, -1e-30, 1e-38, 5.0, 0.25, -0.25, 0.75, -0.75] * 2).to(torch.bfloat16)
    p = torch.ones(k)
    g = laws.svdq_nvfp4_input_scale(x, p)
    assert g.item() == 1.0
    down = torch.zeros(32, k, dtype=torch.bfloat16)
    act, ascales, _ = ops.svdq_quantize(x.to(DEV), p.to(DEV), g.to(DEV), down.to(DEV))
    codes, scales = laws.svdq_nvfp4_quantize(laws.svdq_smooth(x, p), g)
    assert torch.equal(act[:m].cpu(), laws.svdq_nvfp4_pack(codes))
    assert torch.equal(ascales[:m].cpu().view(torch.uint8), scales.view(torch.uint8))


@pytest.mark.parametrize("shape", [(300, 264, 256), (1, 520, 64), (513, 256, 192), (4096, 12288, 64)],
                         ids=lambda s: "x".join(map(str, s)))  # fmt: skip
def test_svdq_gemm_bit_exact_where_exact(ops, shape):
    """Random codes on both sides with E4M3 scales in [1, 2), unit second levels, no c, a zero
    low-rank branch: every product and partial sum is exact in float32 (at most 23 significant
    bits), so the output is the float64 law's, cast once, bit for bit — the fp16 decode of each
    E2M1 code and scale and the MFMA layout, checked exactly. The small grids run 256x192 tiles
    (partial ones past N = 192 or 384), 4096 x 12288 the 256x256 tile (768 tiles: three rounds,
    where 256x192 would need four)."""
    m, n, k = shape
    gen = torch.Generator().manual_seed(m + n + k)
    acodes = torch.randint(0, 16, (m, k), generator=gen).to(torch.uint8)
    wcodes = torch.randint(0, 16, (n, k), generator=gen).to(torch.uint8)
    ascl = torch.randint(0x38, 0x40, (m, k // 16), generator=gen).to(torch.uint8).view(torch.float8_e4m3fn)
    wscl = torch.randint(0x38, 0x40, (n, k // 16), generator=gen).to(torch.uint8).view(torch.float8_e4m3fn)
    padded = -(-m // 256) * 256
    act = torch.zeros(padded, k // 2, dtype=torch.uint8)
    act[:m] = laws.svdq_nvfp4_pack(acodes)
    asc = torch.zeros(padded, k // 16, dtype=torch.uint8)
    asc[:m] = ascl.view(torch.uint8)
    one = torch.ones(1)
    la = torch.zeros(padded, 32, dtype=torch.bfloat16)
    up = torch.zeros(n, 32, dtype=torch.bfloat16)
    exact = laws.svdq_nvfp4_values(acodes, ascl, one).double() @ \
        laws.svdq_nvfp4_values(wcodes, wscl, one).double().t()  # fmt: skip
    for dtype in (torch.bfloat16, torch.float16):
        got = ops.svdq_gemm(act.to(DEV), asc.view(torch.float8_e4m3fn).to(DEV), la.to(DEV), m,
                            one.to(DEV), laws.svdq_nvfp4_pack(wcodes).to(DEV), wscl.to(DEV),
                            one.to(DEV), up.to(DEV), None, None, dtype)  # fmt: skip
        assert torch.equal(got.cpu(), exact.float().to(dtype))


CASES = [(1, 256, 64, 32), (100, 520, 1024, 64), (300, 1032, 2048, 128), (513, 264, 3072, 32),
         (64, 3072, 3072, 32)]


@pytest.mark.parametrize("variant", ["plain", "channel+bias", "stored"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_svdq_linear_within_tolerance(ops, case, dtype, variant):
    m, n, k, r = case
    d = roles(n, k, r, seed=n + k, channel=variant == "channel+bias", stored=variant == "stored")
    x = activations(m, k, seed=m + r, dtype=dtype)
    b = (torch.randn(n, generator=torch.Generator().manual_seed(9)) * 0.1).to(dtype) \
        if variant == "channel+bias" else None  # fmt: skip
    got = ops.svdq_linear(x.to(DEV), on(d), None if b is None else b.to(DEV), dtype)
    assert got.shape == (m, n) and got.dtype == dtype
    assert_close(got, laws.svdq_nvfp4_exact(x, d, b))


def test_c4_shape_svdq_nvfp4(ops):
    """BASELINE config 4's shape (M=4096, K=N=3072, rank 32) on the nvfp4 law: operand bit-exact,
    output within tolerance of the float64 law."""
    m, n, k, r = 4096, 3072, 3072, 32
    d = roles(n, k, r, seed=20261202)
    x = activations(m, k, seed=20261203)
    b = (torch.randn(n, generator=torch.Generator().manual_seed(4)) * 0.1).to(torch.bfloat16)
    dd = on(d)
    g = ops.svdq_input_scale(x.to(DEV), dd["pre_quant_scale"])
    act, ascales, _ = ops.svdq_quantize(x.to(DEV), dd["pre_quant_scale"], g, dd["lowrank_down"])
    want_g = laws.svdq_nvfp4_input_scale(x, d["pre_quant_scale"])
    assert torch.equal(g.cpu().view(torch.int32), want_g.view(torch.int32))
    codes, scales = laws.svdq_nvfp4_quantize(laws.svdq_smooth(x, d["pre_quant_scale"]), want_g)
    assert torch.equal(act.cpu(), laws.svdq_nvfp4_pack(codes))
    assert torch.equal(ascales.cpu().view(torch.uint8), scales.view(torch.uint8))
    got = ops.svdq_linear(x.to(DEV), dd, b.to(DEV), torch.bfloat16)
    assert_close(got, laws.svdq_nvfp4_exact(x, d, b))


# ------------------------------------------------------------------------------ the leaf


class _Linear(torch.nn.Module):
    def __init__(self, bias: torch.Tensor | None) -> None:
        super().__init__()
        self.bias = bias


def _as_stored(d: dict, params: dict) -> dict:
    """The law's roles (`weight` element 2k low, row-major scales, multiply) for stored parts of
    any convention: the nibbles swapped back, the cuBLAS tiles undone (`laws.from_blocked`, held
    by the reference's decode vectors), a divided second level inverted."""
    out = dict(d)
    n, k = int(d["weight"].shape[0]), 2 * int(d["weight"].shape[1])
    if params.get("nibble_order") == "high_first":
        w = d["weight"].view(torch.uint8)
        out["weight"] = (w << 4) | (w >> 4)
    if params.get("scale_layout") == "cublas_128x4":
        grid = laws.from_blocked(d["scale"].view(torch.uint8).reshape(-1), n, k // 16)
        out["scale"] = grid.reshape(n, k // 16).view(torch.float8_e4m3fn)
    second = d["scale_2"].float().reshape(1)
    out["scale_2"] = 1.0 / second if params.get("global_scale") == "divide" else second
    for role in ("channel_scale", "input_scale", "pre_quant_scale"):
        if role in out:
            out[role] = out[role].float()
    return out


def _vector_cases():
    import vectors

    return [c for c in vectors.cases("svdq", "svdq") if "refuse" not in c]


@pytest.mark.parametrize("case", _vector_cases(), ids=lambda c: c["key"])
def test_svdq_leaf_on_reference_vectors(case):
    """The provider's leaf from the reference's own svdq.nvfp4 parts (every stored convention
    the vectors hold: nibble order, cuBLAS tiles, divided second level, E4M3 channel scale, stored
    input scale, fp16 and f32 factors, rank 4 padded to 32) against the float64 law; a case whose
    K is not whole GEMM steps is refused by `supports`."""
    import vectors
    from cozyq import leaves

    parts, params = vectors.parts(case), dict(case["encoding"]["params"])
    provider = leaves.SvdqNvfp4NativeLeaf("svdq.nvfp4", tuple(sorted(params.items())))
    shape = case["shape"]
    why = provider.supports(shape, params)
    if shape[1] % 64:
        assert "K % 64" in why
        return
    assert why == ""
    n, k = shape
    dtype = torch.float16 if case["dtype"] == "F16" else torch.bfloat16
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(n)) * 0.1).to(dtype)
    leaf = provider.leaf(torch, {role: t.to(DEV) for role, t in parts.items()}, _Linear(bias.to(DEV)), dtype)
    x = activations(37, k, seed=k + n, dtype=dtype)
    got = leaf(x.to(DEV))
    assert got.shape == (37, n) and got.dtype == dtype
    law = _as_stored(parts, params)
    law["lowrank_down"], law["lowrank_up"] = law["lowrank_down"].to(torch.bfloat16), law["lowrank_up"].to(torch.bfloat16)
    assert_close(got, laws.svdq_nvfp4_exact(x, law, bias))


def test_svdq_leaf_conventions_and_unbuilt_rank():
    """A larger leaf stored high-first, in cuBLAS tiles, with a divided second level and rank 20
    (padded to 32), in fp16: the leaf against the law on the stored roles."""
    from cozyq import leaves

    n, k, r = 264, 1024, 20
    d = roles(n, k, r, seed=31)
    d["scale_2"] = torch.tensor(50.0)
    stored = dict(d)
    w = d["weight"]
    stored["weight"] = (w << 4) | (w >> 4)
    stored["scale"] = laws.to_blocked(d["scale"].view(torch.uint8)).view(torch.float8_e4m3fn)
    params = (("block_size", 16), ("global_scale", "divide"), ("nibble_order", "high_first"),
              ("scale_layout", "cublas_128x4"))  # fmt: skip
    leaf = leaves.SvdqNvfp4NativeLeaf("svdq.nvfp4", params).leaf(
        torch, {role: t.to(DEV) for role, t in stored.items()}, _Linear(None), torch.float16)  # fmt: skip
    assert int(leaf.lowrank_down.shape[0]) == 32
    x = activations(300, k, seed=32, dtype=torch.float16)
    law = dict(d)
    law["scale_2"] = 1.0 / torch.tensor([50.0])
    assert_close(leaf(x.to(DEV)), laws.svdq_nvfp4_exact(x, law, None))


@pytest.mark.parametrize("extra", [16, 120], ids=["merged", "apart"])
def test_svdq_leaf_lora_branches(extra):
    """A baked request's LoRA (`adopt`): within the kernels' 128 ranks it joins the branch (one
    GEMM); past them it is its own term. Either way the law plus x·Aᵀ·(s·B)ᵀ."""
    from cozyq import leaves

    n, k, r = 264, 512, 32
    d = roles(n, k, r, seed=41)
    leaf = leaves.SvdqNvfp4NativeLeaf().leaf(torch, on(d), _Linear(None), torch.bfloat16)
    gen = torch.Generator().manual_seed(42)
    a = (torch.randn(extra, k, generator=gen) * 0.05).to(torch.bfloat16)
    b = (torch.randn(n, extra, generator=gen) * 0.05).to(torch.bfloat16)
    leaf.adopt(lambda: [("lora", a.to(DEV), b.to(DEV), 0.5)])
    x = activations(64, k, seed=43)
    got = leaf(x.to(DEV))
    want = laws.svdq_nvfp4_exact(x, d, None) + (x.double() @ a.double().t()) @ (0.5 * b.double()).t()
    assert_close(got, want)
    assert (leaf._cozy_merged[1] is None) == (r + extra > 128)


def test_svdq_quantize_and_input_scale_propagate_nan(ops):
    """A NaN in x, as the law treats it (torch's amax and clamp propagate NaN): the block holding
    it gets the E4M3 NaN scale 0x7F and codes 0, + 8 where x < 0 (every threshold comparison with
    a NaN quotient is false); the other blocks are untouched; and the input scale of an x holding
    a NaN is NaN. Held to the oracle bit for bit, at a stored (finite) second level."""
    m, k = 40, 256
    x = activations(m, k, seed=41)
    x[3, 17] = float("nan")
    x[10, 200] = float("nan")
    x[10, 201] = -1.0
    x[10, 202] = 1.0
    d = roles(264, k, 32, seed=42)
    p = d["pre_quant_scale"]
    g = torch.tensor([0.05])
    act, ascales, _ = ops.svdq_quantize(x.to(DEV), p.to(DEV), g.to(DEV), d["lowrank_down"].to(DEV))
    codes, scales = laws.svdq_nvfp4_quantize(laws.svdq_smooth(x, p), g)
    assert scales.view(torch.uint8)[3, 1] == 0x7F and scales.view(torch.uint8)[10, 12] == 0x7F
    assert codes[10, 201] == 8 and codes[10, 202] == 0 and codes[10, 200] == 0
    assert torch.equal(act[:m].cpu(), laws.svdq_nvfp4_pack(codes))
    assert torch.equal(ascales[:m].cpu().view(torch.uint8), scales.view(torch.uint8))
    got = ops.svdq_input_scale(x.to(DEV), p.to(DEV))
    assert torch.isnan(got).all() and torch.isnan(laws.svdq_nvfp4_input_scale(x, p)).all()

"""The LoRA bake (`oracle/bake.py` on the CPU, `csrc/bake.hip` + `cozyq.bake` on the GPU).

CPU: the oracle pinned to things other than itself — Philox's published known-answer vectors,
Triton's own draws (`tests/golden/philox_vectors.json`), exact rational FMA, brute force over
the E4M3 / E2M1 grids, the reference's self-check cases (`internal/lora_bake.py:852-898`),
rank-0 identity and the expectation of stochastic rounding. GPU: every form bit-exact against
the oracle over ragged shapes, ranks and seeds, through the C ABI and the host mirror.
"""

from __future__ import annotations

import math
import json
import random
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import bake as ob
from oracle import laws

GOLDEN = Path(__file__).resolve().parent / "golden"
CUDA = "cuda:0"


# ----------------------------------------------------------------------------- noise pins


@pytest.mark.parametrize("key,counter,want", [
    (0, (0, 0, 0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((1 << 64) - 1, (0xFFFFFFFF,) * 4, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    (0x299F31D0A4093822, (0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
])  # fmt: skip
def test_philox_known_answers(key, counter, want):
    """Random123's published philox4x32-10 known-answer vectors."""
    got = ob.philox(key, *(np.array([c], dtype=np.uint64) for c in counter))
    assert tuple(int(v[0]) for v in got) == want


def test_noise_matches_tritons_draws():
    data = json.loads((GOLDEN / "philox_vectors.json").read_text())
    for case in data["cases"]:
        offsets = np.array(case["offsets"], dtype=np.uint64)
        assert ob.randint(case["seed"], offsets).tolist() == case["randint"], case["seed"]
        bits = ob.rand(case["seed"], offsets).view(np.uint32).tolist()
        assert bits == case["rand_bits"], case["seed"]
        assert (ob.rand(case["seed"], offsets) < 1).all()


# ----------------------------------------------------------------------------- exact FMA


def _round_f32(x: Fraction) -> float:
    """Exact rational → nearest float32 (ties to even), by integer arithmetic."""
    if x == 0:
        return 0.0
    sign, x = (-1.0 if x < 0 else 1.0), abs(x)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    while Fraction(2) ** e > x:
        e -= 1
    while Fraction(2) ** (e + 1) <= x:
        e += 1
    quantum = Fraction(2) ** (max(e, -126) - 23)
    q, r = divmod(x, quantum)
    q = int(q)
    if r * 2 > quantum or (r * 2 == quantum and q % 2 == 1):
        q += 1
    return sign * float(np.float32(float(q * quantum)))


def test_fma32_is_correctly_rounded():
    rng = random.Random(11)
    a, b, c = [], [], []
    for _ in range(3000):
        x = np.float32(rng.uniform(-4, 4) * 2.0 ** rng.randint(-30, 30))
        y = np.float32(rng.uniform(-4, 4) * 2.0 ** rng.randint(-30, 30))
        a.append(x)
        b.append(y)
        # Constructed near-ties: c cancels the product's top, so its low bits decide.
        p = float(x) * float(y)
        choice = rng.randrange(4)
        if choice == 0:
            c.append(np.float32(-p))
        elif choice == 1:
            c.append(np.float32(-p * (1 + 2.0**-24)))
        elif choice == 2:
            c.append(np.float32(p * 2.0**-25))
        else:
            c.append(np.float32(rng.uniform(-4, 4) * 2.0 ** rng.randint(-40, 40)))
    # (1 + 2^-12)^2 - 1: the unfused form loses the 2^-24 term.
    a.append(np.float32(1 + 2.0**-12))
    b.append(np.float32(1 + 2.0**-12))
    c.append(np.float32(-1))
    a, b, c = (np.array(v, dtype=np.float32) for v in (a, b, c))
    got = ob.fma32(a, b, c)
    for i in range(len(a)):
        want = _round_f32(Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i])))
        assert float(got[i]) == want, (a[i], b[i], c[i])
    assert float(got[-1]) == 2.0**-11 + 2.0**-24


# ----------------------------------------------------------------------------- grids


def _e4m3_magnitudes() -> np.ndarray:
    return ob.e4m3_value(np.arange(127))


def test_e4m3_value_against_torch():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = ob.e4m3_value(codes)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite], want[finite])
    assert got[127] == 448 and got[255] == -448


def test_e4m3_stochastic_neighbours():
    """Every grid value rounds to itself under any noise; between two neighbours the result is
    one of them, the upper exactly when the noise's top twenty bits exceed the covered part."""
    mags = _e4m3_magnitudes()
    noise = np.array([0, 1 << 12, 0x7FFFFFFF, 0xFFFFFFFF, 0x12345678], dtype=np.uint32)
    for code in range(127):
        for sign in (1, -1):
            got = ob.e4m3_stochastic(np.full(noise.shape, sign * mags[code], np.float32), noise)
            want = code | (128 if sign < 0 and mags[code] != 0 else 0)
            assert (got == want).all(), (code, sign)
    rng = np.random.default_rng(3)
    for low in range(126):
        frac = rng.random(64).astype(np.float32)
        x = (mags[low] + frac * (mags[low + 1] - mags[low])).astype(np.float32)
        draws = rng.integers(0, 1 << 32, 64, dtype=np.uint64).astype(np.uint32)
        got = ob.e4m3_stochastic(x, draws).astype(np.int64)
        assert set(got.tolist()) <= {low, low + 1}
        # The covered part in units of 2^-20 of a step, against the noise's top 20 bits.
        step = np.float64(mags[low + 1]) - np.float64(mags[low])
        covered = np.floor((x.astype(np.float64) - mags[low]) / step * (1 << 20) + 1e-9)
        up = (draws >> 12).astype(np.float64) + covered >= (1 << 20)
        assert np.array_equal(got == low + 1, up), low
    assert ob.e4m3_stochastic(np.float32([1e6, -1e6, 448.5]), np.uint32([0xFFFFFFFF] * 3)).tolist() == [126, 254, 126]


def test_e4m3_at_least_is_the_least_holding_code():
    mags = _e4m3_magnitudes()
    rng = np.random.default_rng(5)
    need = np.concatenate([mags, mags * np.float32(1 + 2**-20), rng.random(4000).astype(np.float32) * 500,
                           rng.random(1000).astype(np.float32) * 0.02, [0.0]]).astype(np.float32)  # fmt: skip
    got = ob.e4m3_at_least(need)
    want = np.minimum(np.searchsorted(mags, need, side="left"), 126)
    assert np.array_equal(got, want)


def test_e2m1_value_and_stochastic():
    assert ob.e2m1_value(np.arange(16)).tolist() == [0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6]
    grid = ob.e2m1_value(np.arange(8))
    for code in range(8):
        for draw in (0.0, 0.5, 0.999):
            assert int(ob.e2m1_stochastic(np.float32([grid[code]]), np.float32([draw]))[0]) == code
    rng = np.random.default_rng(6)
    for low in range(7):
        x = (grid[low] + rng.random(200) * (grid[low + 1] - grid[low])).astype(np.float32)
        draw = rng.random(200).astype(np.float32)
        got = ob.e2m1_stochastic(x, draw)
        frac = (x - grid[low]) / (grid[low + 1] - grid[low])
        assert np.array_equal(got, low + (draw < frac)), low
    assert ob.e2m1_stochastic(np.float32([7.0, -100.0]), np.float32([0.0, 0.9])).tolist() == [7, 7]


# ----------------------------------------------------------------------------- bakes


def _probe_factors(rows: int = 70, rank: int = 24, cols: int = 96):
    up = np.full((rows, rank), 1 / 32, dtype=np.float32)
    up[1::2] = -1 / 32
    return up, np.ones((rank, cols), dtype=np.float32)


def _want(rows: int, cols: int) -> np.ndarray:
    return np.tile(np.float32([[1.0], [-0.5]]), (rows // 2, cols))


def _bf16_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _decode(form: int, data: np.ndarray, scale=None) -> np.ndarray:
    if form == ob.BF16:
        return (data.astype(np.uint32) << 16).view(np.float32)
    if form == ob.F16:
        return data.view(np.float16).astype(np.float32)
    if form == ob.ROWWISE:
        return ob.e4m3_value(data) * scale.reshape(-1, 1)
    if form == ob.INT8:
        return data.astype(np.float32) * scale.reshape(-1, 1)
    return data.astype(np.float32)


@pytest.mark.parametrize("form", [ob.BF16, ob.F16, ob.F32, ob.ROWWISE])
def test_reference_self_check_cases(form):
    """`probe`: 0.25 + 24·(±1/32) is 1.0 or −0.5 on every grid, over partial tiles."""
    rows, cols = 70, 96
    up, down = _probe_factors()
    if form == ob.ROWWISE:
        data = np.full((rows, cols), 0x30, dtype=np.uint8)  # E4M3 0.5
        scale = np.full(rows, 0.5, dtype=np.float32)
    else:
        quarter = np.full((rows, cols), 0.25, dtype=np.float32)
        data = {ob.BF16: _bf16_bits(quarter), ob.F16: quarter.astype(np.float16).view(np.uint16),
                ob.F32: quarter}[form]  # fmt: skip
        scale = None
    out = ob.bake(form, data, scale, up, down, form)
    assert np.array_equal(_decode(form, out, scale), _want(rows, cols))


def test_reference_self_check_nvfp4_and_int8():
    rows, cols = 70, 96
    up, down = _probe_factors()
    codes, blocks = ob.bake_nvfp4(np.full((rows, cols // 2), 0x11, np.uint8),
                                  np.full((rows, cols // 16), 0x30, np.uint8), 1.0, up, down, 5)  # fmt: skip
    assert (blocks == 0x30).all()
    nib = np.stack((codes & 15, codes >> 4), -1).reshape(rows, cols)
    assert np.array_equal(ob.e2m1_value(nib) * 0.5, _want(rows, cols))
    # int8 of rotated rows: 2 + 24·(±1/48)/0.5 is 3 or 1; H keeps a constant row.
    ones = np.ones((24, 256), dtype=np.float32)
    assert np.array_equal(ob.rotate_factor(ones), ones)
    out = ob.bake(ob.INT8, np.full((rows, 256), 2, np.int8), np.full(rows, 0.5, np.float32),
                  up * np.float32(32 / 48), ob.rotate_factor(ones), 4)  # fmt: skip
    assert np.array_equal(out, np.tile(np.int8([[3], [1]]), (rows // 2, 256)))


def test_rotate_factor_is_orthonormal():
    rng = np.random.default_rng(8)
    x = rng.integers(-50, 50, (3, 512)).astype(np.float32)
    assert np.array_equal(ob.rotate_factor(ob.rotate_factor(x)), x)
    y = rng.standard_normal((4, 768)).astype(np.float32)
    r = ob.rotate_factor(y)
    np.testing.assert_allclose(np.linalg.norm(r, axis=1), np.linalg.norm(y, axis=1), rtol=1e-5)


def _random_stored(form: int, rows: int, cols: int, rng):
    w = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    if form == ob.BF16:
        return _bf16_bits(w), None
    if form == ob.F16:
        return w.astype(np.float16).view(np.uint16), None
    if form == ob.F32:
        return w, None
    # Headroom under the grid's top (448, 127) so that a small delta never saturates.
    scale = (np.abs(w).max(axis=1) / (400.0 if form == ob.ROWWISE else 110.0)).astype(np.float32)
    if form == ob.ROWWISE:
        data = torch.from_numpy(w / scale[:, None]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        return data, scale
    return np.clip(np.rint(w / scale[:, None]), -127, 127).astype(np.int8), scale


@pytest.mark.parametrize("form", [ob.BF16, ob.F16, ob.F32, ob.ROWWISE, ob.INT8])
def test_rank_zero_writes_every_byte_back(form):
    rng = np.random.default_rng(form)
    data, scale = _random_stored(form, 9, 40, rng)
    if form == ob.ROWWISE:
        data[0, :4] = [0x7F, 0xFF, 0x80, 0x00]  # reserved codes saturate; −0 becomes +0
    out = ob.bake(form, data, scale, np.zeros((9, 0), np.float32), np.zeros((0, 40), np.float32), 3)
    want = data.copy()
    if form == ob.ROWWISE:
        want[0, :4] = [0x7E, 0xFE, 0x00, 0x00]
    assert np.array_equal(out.view(np.uint8), want.view(np.uint8))
    codes = rng.integers(0, 256, (9, 16), dtype=np.uint8)
    blocks = rng.integers(1, 100, (9, 2), dtype=np.uint8)
    got = ob.bake_nvfp4(codes, blocks, 0.01, np.zeros((9, 0), np.float32), np.zeros((0, 32), np.float32), 1)
    assert np.array_equal(got[0], codes) and np.array_equal(got[1], blocks)


@pytest.mark.parametrize("form", [ob.BF16, ob.ROWWISE, ob.INT8])
def test_stochastic_bake_is_unbiased(form):
    """The mean over seeds of the stored value is the exact target, within the sampling bound."""
    rng = np.random.default_rng(20 + form)
    rows, cols, rank = 4, 64, 3
    data, scale = _random_stored(form, rows, cols, rng)
    up = (rng.standard_normal((rows, rank)) * 0.01).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    used = ob.rotate_factor(np.pad(down, ((0, 0), (0, 256 - cols)))) if form == ob.INT8 else down
    if form == ob.INT8:
        data = np.pad(data, ((0, 0), (0, 256 - cols)))
    base = _decode(form, data, scale).astype(np.float64)
    target = base + up.astype(np.float64) @ used.astype(np.float64)
    seeds = 400
    total = sum(_decode(form, ob.bake(form, data, scale, up, used, s), scale).astype(np.float64)
                for s in range(seeds))  # fmt: skip
    mean = total / seeds
    # One step of the grid bounds a single draw's error; the mean's spread is ≤ step/(2√seeds).
    if form == ob.BF16:
        step = np.abs(target) * 2.0**-7
    elif form == ob.ROWWISE:
        step = np.maximum(np.abs(target) * 2.0**-3, 2.0**-9 * scale[:, None])
    else:
        step = np.broadcast_to(scale[:, None].astype(np.float64), target.shape)
    assert (np.abs(mean - target) <= 5 * step / (2 * np.sqrt(seeds)) + 1e-12).all()


def test_nvfp4_block_grows_past_seven_sixths():
    """A block whose baked maximum passes 7/6 of its scale takes the least code that holds it;
    one under that keeps its scale and saturates."""
    rows, cols = 2, 16
    codes = np.full((rows, 8), 0x77, np.uint8)  # every element 6
    blocks = np.full((rows, 1), 0x38, np.uint8)  # E4M3 1.0
    up = np.float32([[0.9], [1.5]])  # 6 + 0.9 < 7 (kept); 6 + 1.5 > 7 (grows)
    down = np.ones((1, cols), np.float32)
    new_codes, new_blocks = ob.bake_nvfp4(codes, blocks, 1.0, up, down, 9)
    assert new_blocks[0, 0] == 0x38 and (new_codes[0] == 0x77).all()
    need = np.float32(7.5) / np.float32(6)
    grown = int(new_blocks[1, 0])
    assert grown == int(ob.e4m3_at_least(np.float32([need]))[0])
    assert ob.e4m3_value(grown) >= need > ob.e4m3_value(grown - 1)


def test_f16_rounds_to_nearest():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((5, 24)) * 0.1).astype(np.float16)
    up = np.float32(rng.integers(-8, 8, (5, 1))) * np.float32(2.0**-12)
    down = np.ones((1, 24), np.float32)
    out = ob.bake(ob.F16, w.view(np.uint16), None, up, down, 0)
    want = (w.astype(np.float64) + up.astype(np.float64)).astype(np.float16)
    assert np.array_equal(out.view(np.float16), want)


# ----------------------------------------------------------------------------- host surface (CPU)


def test_bakeable_mirrors_the_reference_roles():
    from cozyq import bake as cb

    assert cb.bakeable("plain", {}, {"value": "bf16"})
    assert not cb.bakeable("plain", {}, {"value": "f8_e4m3fn"})
    assert cb.bakeable("fp8.rowwise", {}, {"weight": "f8_e4m3fn", "scale": "f32"})
    assert not cb.bakeable("fp8.rowwise", {}, {"weight": "f8_e4m3fn", "scale": "bf16"})
    roles = {"weight": "u8", "scale": "f8_e4m3fn", "scale_2": "f32", "input_scale": "f32"}
    assert cb.bakeable("nvfp4", dict(cb.NVFP4_PARAMS), roles)
    assert not cb.bakeable("nvfp4", {**cb.NVFP4_PARAMS, "scale_layout": "cublas_128x4"}, roles)
    assert not cb.bakeable("nvfp4", {"nibble_order": "high_first"}, roles)
    assert cb.bakeable("int8.convrot", {}, {"weight": "i8", "scale": "f32"})
    assert cb.bakeable("int8.convrot", {"rotation_size": 256}, {"weight": "i8", "scale": "f32"})
    assert not cb.bakeable("int8.convrot", {"rotation_size": 64}, {"weight": "i8", "scale": "f32"})
    assert not cb.bakeable("int8.rowwise", {}, {"weight": "i8", "scale": "f32"})


def test_bake_refuses_what_it_does_not_build():
    from cozyq import bake as cb

    value = torch.zeros(4, 8, dtype=torch.bfloat16)
    down, up = torch.zeros(2, 8), torch.zeros(4, 2)
    with pytest.raises(ValueError, match="GPU"):
        cb.bake(torch, {"value": value}, down, up, seed=1, stats=cb.Stats())
    with pytest.raises(ValueError, match="no bake path"):
        cb.bake(torch, {"value": value}, down, up, seed=1, how="triton")
    for kwargs in ({}, {"how": "eager"}, {"gain": torch.ones(4)}, {"more": lambda a, b: torch.zeros(b - a, 8)}):
        with pytest.raises(ValueError, match="GPU"):
            cb.bake(torch, {"value": value}, down, up, seed=1, **kwargs)
    with pytest.raises(NotImplementedError):
        cb.recipe(False)
    assert cb.recipe().startswith(cb.VARIANT)


def test_abi_refuses_bad_bake_options():
    """Argument checks answer before any device work: a gain on a row-scaled form, unknown
    flags, nvfp4 columns off the 16-block, an unknown form."""
    from cozyq import _lib

    lib = _lib.load()
    bad = lib.cozyq_bake(0, 3, 16, 16, 16, 16, 16, None, None, 4, 8, 2, 1, 0, None)
    assert bad != 0
    assert lib.cozyq_bake(0, 0, 16, None, 16, 16, None, None, None, 4, 8, 2, 1, 4, None) != 0
    assert lib.cozyq_bake(0, 6, 16, None, 16, 16, None, None, None, 4, 8, 2, 1, 0, None) != 0
    # A new row scale is for fp8.rowwise only, and not with "no delta".
    assert lib.cozyq_bake(0, 4, 16, 16, 16, 16, None, None, 16, 4, 256, 2, 1, 0, None) != 0
    assert lib.cozyq_bake(0, 3, 16, 16, 16, 16, None, None, 16, 4, 8, 2, 1, 2, None) != 0
    assert lib.cozyq_bake_row_amax(0, 7, 16, None, None, None, 16, 16, None, None, 4, 8, 2, 16, None) != 0
    assert lib.cozyq_bake_nvfp4(0, 16, 16, 16, 16, 16, None, None, 4, 24, 2, 1, 0, None) != 0
    assert lib.cozyq_bake_norms(0, 6, 16, None, None, None, 16, 16, 4, 8, 2, 16, None) != 0
    assert lib.cozyq_bake_rotate_factor(0, 16, 16, 2, 100, None) != 0
    # nvfp4 refit: a positive finite level, nearest or stochastic only, 16-column blocks.
    assert lib.cozyq_bake_nvfp4_refit(0, 16, 16, 16, 0.0, 16, 16, None, None, 4, 32, 2, 1, 0, None) != 0
    assert lib.cozyq_bake_nvfp4_refit(0, 16, 16, 16, float("inf"), 16, 16, None, None, 4, 32, 2, 1, 0, None) != 0
    assert lib.cozyq_bake_nvfp4_refit(0, 16, 16, 16, 1.0, 16, 16, None, None, 4, 32, 2, 1, 2, None) != 0
    assert lib.cozyq_bake_nvfp4_refit(0, 16, 16, 16, 1.0, 16, 16, None, None, 4, 24, 2, 1, 0, None) != 0
    # A gain belongs to the plain and nvfp4 forms' row maxima only.
    assert lib.cozyq_bake_row_amax(0, 3, 16, 16, None, None, 16, 16, 16, None, 4, 8, 2, 16, None) != 0
    # Empty shapes succeed without touching a device.
    assert lib.cozyq_bake(0, 0, None, None, None, None, None, None, None, 0, 8, 2, 1, 0, None) == 0


def test_nearest_grids_tie_to_even():
    mags = _e4m3_magnitudes()
    mids = ((mags[:-1].astype(np.float64) + mags[1:]) / 2).astype(np.float32)
    got = ob.e4m3_nearest(mids).astype(np.int64)
    low = np.arange(126)
    assert np.array_equal(got, np.where(low % 2 == 0, low, low + 1))
    rng = np.random.default_rng(12)
    x = (rng.random(5000) * 460).astype(np.float32)
    near = np.argmin(np.abs(mags[None, :].astype(np.float64) - x[:, None]), axis=1)
    got = ob.e4m3_nearest(x).astype(np.int64)
    assert (np.abs(mags[got] - x) <= np.abs(mags[near] - x)).all()
    assert ob.e4m3_nearest(np.float32([-0.0, -1.0, -500.0])).tolist() == [0, 0xB8, 0xFE]
    grid = ob.e2m1_value(np.arange(8))
    mid2 = ((grid[:-1] + grid[1:]) / 2).astype(np.float32)
    assert ob.e2m1_nearest(mid2).tolist() == [0, 2, 2, 4, 4, 6, 6]
    assert ob.e2m1_nearest(np.float32([0.2, 0.3, 5.1, 9.0])).tolist() == [0, 1, 7, 7]


def test_gain_rows_laws():
    """`gain_rows` on plain rows is the reference's own line, `value.float() * gain` cast to
    nearest; on nvfp4 rows a unit gain writes every byte back."""
    rng = np.random.default_rng(13)
    w = (rng.standard_normal((6, 40)) * 0.1).astype(np.float32)
    gain = (rng.random(6) + 0.5).astype(np.float32)
    bits = _bf16_bits(w)
    got = ob.bake(ob.BF16, bits, None, np.zeros((6, 0), np.float32), np.zeros((0, 40), np.float32), 0,
                  gain=gain, nearest=True, no_delta=True)  # fmt: skip
    want = (torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float() * torch.from_numpy(gain)[:, None]
            ).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)  # fmt: skip
    assert np.array_equal(got, want)
    codes = rng.integers(0, 256, (6, 16), dtype=np.uint8)
    blocks = rng.integers(0x28, 0x48, (6, 2), dtype=np.uint8)
    none_r, none_c = np.zeros((6, 0), np.float32), np.zeros((0, 32), np.float32)
    same = ob.bake_nvfp4(codes, blocks, 0.05, none_r, none_c, 0, gain=np.ones(6, np.float32),
                         nearest=True, no_delta=True)  # fmt: skip
    assert np.array_equal(same[0], codes) and np.array_equal(same[1], blocks)


@pytest.mark.parametrize("form", [ob.BF16, ob.F16, ob.F32, ob.ROWWISE, ob.INT8, ob.NVFP4])
def test_norms_against_float64(form):
    rng = np.random.default_rng(40 + form)
    rows, cols, rank = 7, 256, 3
    up = (rng.standard_normal((rows, rank)) * 0.05).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    if form == ob.NVFP4:
        codes = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
        blocks = rng.integers(0x28, 0x48, (rows, cols // 16), dtype=np.uint8)
        got = ob.norms(form, codes, None, up, down, blocks=blocks, second=0.02)
        nib = np.stack((codes & 15, codes >> 4), -1).reshape(rows, cols)
        s = torch.from_numpy(np.repeat(blocks, 16, axis=1)).view(torch.float8_e4m3fn).double().numpy()
        base = np.asarray(laws_values(nib), np.float64) * s * 0.02
    else:
        data, scale = _random_stored(form, rows, cols, rng)
        got = ob.norms(form, data, scale, up, down)
        base = _decode(form, data, scale).astype(np.float64)
    want = np.linalg.norm(base + up.astype(np.float64) @ down.astype(np.float64), axis=1)
    np.testing.assert_allclose(got, want, rtol=2e-6)


def laws_values(nib: np.ndarray) -> np.ndarray:
    table = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6])
    return table[nib.astype(np.int64)]


# ----------------------------------------------------------------------------- GPU parity


def _stored_for(form: int, rows: int, cols: int, seed: int):
    rng = np.random.default_rng(seed)
    data, scale = _random_stored(form, rows, cols, rng)
    if form == ob.INT8:
        data = np.ascontiguousarray(data)
    return data, scale, rng


def _torch_data(form: int, data: np.ndarray) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(data))
    return {ob.BF16: lambda: t.view(torch.bfloat16), ob.F16: lambda: t.view(torch.float16),
            ob.F32: lambda: t, ob.ROWWISE: lambda: t, ob.INT8: lambda: t}[form]()  # fmt: skip


def _bytes(t: torch.Tensor) -> np.ndarray:
    return t.cpu().contiguous().view(torch.uint8).numpy()


SHAPES = [(70, 96, 24), (1, 1, 1), (129, 257, 33), (64, 128, 0), (300, 1000, 64), (3, 4, 40)]


@pytest.mark.gpu
@pytest.mark.parametrize("form", [ob.BF16, ob.F16, ob.F32, ob.ROWWISE])
@pytest.mark.parametrize("rows,cols,rank", SHAPES)
def test_gpu_bake_bit_exact(form, rows, cols, rank):
    from cozyq import prebuilt

    print(f"bake form={form} rows={rows} cols={cols} rank={rank}", flush=True)
    data, scale, rng = _stored_for(form, rows, cols, 100 * form + rows)
    up = (rng.standard_normal((rows, rank)) * 0.02).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    seed = int(rng.integers(0, 1 << 31))
    want = ob.bake(form, data, scale, up, down, seed)
    ops = prebuilt.library(0)
    t = _torch_data(form, data).to(CUDA)
    s = None if scale is None else torch.from_numpy(scale).to(CUDA)
    ops.bake(form, t, s, torch.from_numpy(up).to(CUDA), torch.from_numpy(down).to(CUDA), seed)
    torch.cuda.synchronize()
    assert np.array_equal(_bytes(t), want.view(np.uint8).reshape(rows, -1))


@pytest.mark.gpu
@pytest.mark.parametrize("form", [ob.BF16, ob.ROWWISE])
def test_gpu_bake_unaligned_rows_and_high_seed(form):
    """A data pointer off its four-element alignment takes the element path; a seed with bit 31
    set keys Philox with the sign-extended word, as an int32 Triton argument does."""
    from cozyq import prebuilt

    rows, cols, rank = 33, 64, 5
    data, scale, rng = _stored_for(form, rows, cols + 1, 7 + form)
    up = (rng.standard_normal((rows, rank)) * 0.02).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    seed = 0x80000123
    backing = _torch_data(form, data).to(CUDA)
    view = backing.view(-1)[1 : 1 + rows * cols].view(rows, cols)  # offset by one element
    host = _bytes(view).view(data.dtype).reshape(rows, cols)
    want = ob.bake(form, host, scale, up, down, seed)
    prebuilt.library(0).bake(form, view, None if scale is None else torch.from_numpy(scale).to(CUDA),
                             torch.from_numpy(up).to(CUDA), torch.from_numpy(down).to(CUDA), seed)  # fmt: skip
    torch.cuda.synchronize()
    assert np.array_equal(_bytes(view), want.view(np.uint8).reshape(rows, -1))


@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols,rank", [(70, 256, 24), (129, 512, 33), (5, 1024, 7), (64, 256, 0)])
def test_gpu_bake_int8_convrot_bit_exact(rows, cols, rank):
    from cozyq import bake as cb

    print(f"bake int8 rows={rows} cols={cols} rank={rank}", flush=True)
    data, scale, rng = _stored_for(ob.INT8, rows, cols, rows + rank)
    up = (rng.standard_normal((rows, rank)) * 0.02).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    seed = int(rng.integers(0, 1 << 31))
    rotated = cb.rotate_factor(torch, torch.from_numpy(down).to(CUDA))
    assert np.array_equal(rotated.cpu().numpy().view(np.uint32), ob.rotate_factor(down).view(np.uint32))
    want = ob.bake(ob.INT8, data, scale, up, ob.rotate_factor(down), seed)
    stored = {"weight": torch.from_numpy(data).to(CUDA), "scale": torch.from_numpy(scale).to(CUDA)}
    cb.bake(torch, stored, torch.from_numpy(down).to(CUDA), torch.from_numpy(up).to(CUDA), seed=seed)
    torch.cuda.synchronize()
    assert np.array_equal(stored["weight"].cpu().numpy(), want)


def _nvfp4_stored(rows: int, cols: int, rng):
    codes = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
    blocks = rng.integers(0x20, 0x48, (rows, cols // 16), dtype=np.uint8)  # E4M3 0.125 .. 2.0
    return codes, blocks


@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols,rank,gain", [(70, 96, 24, 0.3), (129, 272, 33, 3.0),
                                                 (300, 1024, 64, 1.0), (16, 16, 0, 1.0),
                                                 (65, 144, 1, 20.0)])  # fmt: skip
def test_gpu_bake_nvfp4_bit_exact(rows, cols, rank, gain):
    """Codes and block bytes bit-exact against the oracle; `gain` sizes the delta so that some
    blocks keep their scale and others grow."""
    from cozyq import bake as cb

    print(f"bake nvfp4 rows={rows} cols={cols} rank={rank}", flush=True)
    rng = np.random.default_rng(rows * cols + rank)
    codes, blocks = _nvfp4_stored(rows, cols, rng)
    second = np.float32(0.03)
    up = (rng.standard_normal((rows, rank)) * 0.02 * gain).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    seed = int(rng.integers(0, 1 << 31))
    want_codes, want_blocks = ob.bake_nvfp4(codes, blocks, second, up, down, seed)
    stored = {"weight": torch.from_numpy(codes).to(CUDA),
              "scale": torch.from_numpy(blocks).view(torch.float8_e4m3fn).to(CUDA),
              "scale_2": torch.tensor([second], device=CUDA)}  # fmt: skip
    cb.bake(torch, stored, torch.from_numpy(down).to(CUDA), torch.from_numpy(up).to(CUDA), seed=seed)
    torch.cuda.synchronize()
    assert np.array_equal(stored["scale"].view(torch.uint8).cpu().numpy(), want_blocks)
    assert np.array_equal(stored["weight"].cpu().numpy(), want_codes)
    if gain >= 3.0:
        assert (want_blocks != blocks).any()


@pytest.mark.gpu
def test_gpu_probe_and_conv_flattening():
    from cozyq import bake as cb

    verdict = cb.probe(torch, torch.device(CUDA))
    assert verdict.ok, verdict.detail
    # A 3x3 convolution bakes as a matrix with 9 columns per input channel.
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((8, 4, 3, 3)) * 0.1).astype(np.float32)
    down = rng.standard_normal((2, 4, 3, 3)).astype(np.float32)
    up = (rng.standard_normal((8, 2, 1, 1)) * 0.1).astype(np.float32)
    want = ob.bake(ob.F32, w.reshape(8, -1), None, up.reshape(8, 2), down.reshape(2, -1), 17)
    stored = {"value": torch.from_numpy(w).to(CUDA)}
    cb.bake(torch, stored, torch.from_numpy(down).to(CUDA), torch.from_numpy(up).to(CUDA), seed=17)
    assert np.array_equal(stored["value"].cpu().numpy().reshape(8, -1), want)


@pytest.mark.gpu
def test_gpu_dora_gain_folds_into_a_row_scale():
    from cozyq import bake as cb

    rows, cols = 16, 64
    data, scale, rng = _stored_for(ob.ROWWISE, rows, cols, 3)
    gain = (rng.random(rows) + 0.5).astype(np.float32)
    stored = {"weight": torch.from_numpy(data).view(torch.float8_e4m3fn).to(CUDA),
              "scale": torch.from_numpy(scale).to(CUDA)}  # fmt: skip
    zero_down, zero_up = torch.zeros(0, cols, device=CUDA), torch.zeros(rows, 0, device=CUDA)
    cb.bake(torch, stored, zero_down, zero_up, seed=1, gain=torch.from_numpy(gain).to(CUDA))
    assert np.array_equal(stored["scale"].cpu().numpy(), scale * gain)
    assert np.array_equal(stored["weight"].view(torch.uint8).cpu().numpy(), data)


@pytest.mark.gpu
def test_gpu_bake_full_size_bf16_properties():
    """At a 4096 x 4096 weight: each baked value is one of the two bf16 neighbours of its exact
    target (within one float32 rounding of the delta) and the mean error over 16M elements is
    centred; a rank-0 bake writes every byte back."""
    from cozyq import prebuilt

    rows = cols = 4096
    rank = 32
    g = torch.Generator(device=CUDA).manual_seed(5)
    base = (torch.randn(rows, cols, device=CUDA, generator=g) * 0.02).to(torch.bfloat16)
    up = torch.randn(rows, rank, device=CUDA, generator=g) * 1e-3
    down = torch.randn(rank, cols, device=CUDA, generator=g)
    ops = prebuilt.library(0)
    data = base.clone()
    ops.bake(ob.BF16, data, None, up, down, 99)
    delta = up.double() @ down.double()
    target = base.double() + delta
    err = data.double() - target
    # The float32 sum the kernel rounds is within `slack` of the exact target: the FMA chain's
    # error is relative to Σ|up·down| (rank roundings), the add's to |base|. A bf16 neighbour of
    # that sum is under one ulp, at most 2^-7 of its magnitude, away.
    slack = (base.double().abs() + up.double().abs() @ down.double().abs()) * 2.0**-17
    ulp = (target.abs() + slack) * 2.0**-7
    excess = err.abs() / (ulp + slack)
    worst = int(excess.argmax())
    assert float(excess.max()) <= 1.0, (
        f"element {worst}: stored {float(data.view(-1)[worst])}, target {float(target.view(-1)[worst])}, "
        f"base {float(base.view(-1)[worst])}, excess {float(excess.max())}")
    assert abs(float(err.mean())) < 4 * float(ulp.mean()) / (rows * cols) ** 0.5
    same = base.clone()
    ops.bake(ob.BF16, same, None, up[:, :0].contiguous(), down[:0].contiguous(), 99)
    assert torch.equal(same.view(torch.int16), base.view(torch.int16))


# ----------------------------------------------------------------------------- GPU: eager additions

EXTRA = [  # (gain, more, nearest, no_delta)
    (True, False, False, False), (False, True, False, False), (True, True, True, False),
    (True, False, True, True), (False, False, True, False),
]


def _extras(rng, rows: int, cols: int, gain: bool, more: bool):
    g = (rng.random(rows) + 0.5).astype(np.float32) if gain else None
    m = (rng.standard_normal((rows, cols)) * 0.01).astype(np.float32) if more else None
    return g, m


def _flags(nearest: bool, no_delta: bool) -> int:
    return (1 if nearest else 0) | (2 if no_delta else 0)


def _cuda(a):
    return None if a is None else torch.from_numpy(a).to(CUDA)


# A row-scaled weight takes its gain in its scale: the kernel's gain is for plain rows only.
OPTION_CASES = [(form, *extra) for form in (ob.BF16, ob.F16, ob.F32, ob.ROWWISE, ob.INT8) for extra in EXTRA
                if not (extra[0] and form in (ob.ROWWISE, ob.INT8))]  # fmt: skip


@pytest.mark.gpu
@pytest.mark.parametrize("form,gain,more,nearest,no_delta", OPTION_CASES)
def test_gpu_bake_options_bit_exact(form, gain, more, nearest, no_delta):
    """gain (plain rows), dense extra rows, nearest rounding and no-delta through the C ABI,
    bit-exact against the oracle, on a ragged shape."""
    from cozyq import prebuilt

    rows, cols, rank = 67, 256 if form == ob.INT8 else 131, 9
    data, scale, rng = _stored_for(form, rows, cols, 500 + form)
    up = (rng.standard_normal((rows, rank)) * 0.02).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    g, m = _extras(rng, rows, cols, gain, more)
    seed = int(rng.integers(0, 1 << 31))
    want = ob.bake(form, data, scale, up, down, seed, gain=g, more=m, nearest=nearest, no_delta=no_delta)
    t = _torch_data(form, data).to(CUDA)
    prebuilt.library(0).bake(form, t, _cuda(scale), _cuda(up), _cuda(down), seed, gain=_cuda(g), more=_cuda(m),
                             flags=_flags(nearest, no_delta))  # fmt: skip
    torch.cuda.synchronize()
    assert np.array_equal(_bytes(t), want.view(np.uint8).reshape(rows, -1))


@pytest.mark.gpu
@pytest.mark.parametrize("gain,more,nearest,no_delta", EXTRA)
def test_gpu_bake_nvfp4_options_bit_exact(gain, more, nearest, no_delta):
    from cozyq import prebuilt

    rows, cols, rank = 70, 272, 5
    rng = np.random.default_rng(71 + 2 * gain + more)
    codes, blocks = _nvfp4_stored(rows, cols, rng)
    up = (rng.standard_normal((rows, rank)) * 0.05).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    g, m = _extras(rng, rows, cols, gain, more)
    if g is not None:
        g = g * 1.5  # some blocks outgrow their scale
    seed = int(rng.integers(0, 1 << 31))
    want = ob.bake_nvfp4(codes, blocks, 0.03, up, down, seed, gain=g, more=m, nearest=nearest, no_delta=no_delta)
    c, b = torch.from_numpy(codes).to(CUDA), torch.from_numpy(blocks).to(CUDA)
    prebuilt.library(0).bake_nvfp4(c, b, torch.tensor([0.03], device=CUDA), _cuda(up), _cuda(down), seed,
                                   gain=_cuda(g), more=_cuda(m), flags=_flags(nearest, no_delta))  # fmt: skip
    torch.cuda.synchronize()
    assert np.array_equal(b.cpu().numpy(), want[1])
    assert np.array_equal(c.cpu().numpy(), want[0])


@pytest.mark.gpu
@pytest.mark.parametrize("form", [ob.BF16, ob.F16, ob.F32, ob.ROWWISE, ob.INT8, ob.NVFP4])
def test_gpu_norms_against_the_oracle(form):
    """`norms` through the host mirror: float64 sums in a fixed order, so equal to the oracle's
    within float64 reassociation, and the same bits on every call."""
    from cozyq import bake as cb

    rng = np.random.default_rng(90 + form)
    rows, cols, rank = 131, 512, 7
    up = (rng.standard_normal((rows, rank)) * 0.05).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    if form == ob.NVFP4:
        codes, blocks = _nvfp4_stored(rows, cols, rng)
        want = ob.norms(form, codes, None, up, down, blocks=blocks, second=0.02)
        stored = {"weight": torch.from_numpy(codes).to(CUDA),
                  "scale": torch.from_numpy(blocks).view(torch.float8_e4m3fn).to(CUDA),
                  "scale_2": torch.tensor([0.02], device=CUDA)}  # fmt: skip
    else:
        data, scale, _ = _stored_for(form, rows, cols, 91 + form)
        used = ob.rotate_factor(down) if form == ob.INT8 else down
        want = ob.norms(form, data, scale, up, used)
        t = _torch_data(form, data).to(CUDA)
        if form in (ob.BF16, ob.F16, ob.F32):
            stored = {"value": t}
        else:
            weight = t.view(torch.float8_e4m3fn) if form == ob.ROWWISE else t
            stored = {"weight": weight, "scale": torch.from_numpy(scale).to(CUDA)}
    got = cb.norms(torch, stored, _cuda(down), _cuda(up))
    again = cb.norms(torch, stored, _cuda(down), _cuda(up))
    assert torch.equal(got, again)
    np.testing.assert_allclose(got.cpu().numpy(), want, rtol=1e-6)


@pytest.mark.gpu
def test_gpu_dora_and_gain_rows_through_the_mirror():
    """`dora` as PEFT's merged weight: with t = 1, baking `c·B @ A` after `gain_rows(g)` lands
    within bf16 rounding of `dora_weight` (float64 reference), for a plain bf16 weight."""
    from cozyq import bake as cb

    rows, cols, rank = 96, 256, 4
    g = torch.Generator().manual_seed(3)
    w = (torch.randn(rows, cols, generator=g) * 0.05).to(torch.bfloat16)
    down = torch.randn(rank, cols, generator=g) * 0.1
    up = torch.randn(rows, rank, generator=g) * 0.1
    magnitude = torch.rand(rows, generator=g) + 0.5
    s, t = 0.8, 1.0
    stored = {"value": w.to(CUDA)}
    gain, scales = cb.dora(torch, stored, [(down.to(CUDA), up.to(CUDA), magnitude.to(CUDA), s, t)])
    cb.gain_rows(torch, stored, gain)
    cb.bake(torch, stored, down.to(CUDA), (up.to(CUDA) * scales[0][:, None]), seed=5)
    want = cb.dora_weight(torch, w.double(), down.double(), up.double(), magnitude.double(), s, t)
    got = stored["value"].double().cpu()
    # Two bf16 roundings: `gain_rows` rounds g·W to nearest (half an ulp of |g·W|), the bake
    # rounds the sum stochastically (under one ulp of it); an ulp is at most 2^-7 of a magnitude.
    scaled = (gain.double().cpu()[:, None] * w.double()).abs()
    bound = (0.5 * scaled + want.abs() + scaled * 2.0**-7) * 2.0**-7 * 1.01 + 1e-6
    assert bool(((got - want).abs() <= bound).all())
    # The row gain on a row-scaled weight is its scale's, exactly.
    data, scale, _ = _stored_for(ob.ROWWISE, rows, cols, 6)
    fp8 = {"weight": torch.from_numpy(data).view(torch.float8_e4m3fn).to(CUDA),
           "scale": torch.from_numpy(scale).to(CUDA)}  # fmt: skip
    cb.gain_rows(torch, fp8, gain)
    assert torch.equal(fp8["scale"].cpu(), torch.from_numpy(scale) * gain.cpu())


@pytest.mark.gpu
@pytest.mark.parametrize("form", [ob.BF16, ob.INT8, ob.NVFP4])
def test_gpu_lokr_rows_bake_bit_exact(form):
    """A LoKr term's dense rows (`Kron`, `dense`) add to the delta; int8.convrot rotates them."""
    from cozyq import bake as cb

    rng = np.random.default_rng(33 + form)
    rows, cols, rank = 64, 256, 3
    w1 = rng.standard_normal((8, 16)).astype(np.float32)
    w2 = rng.standard_normal((8, 16)).astype(np.float32)
    kron = cb.Kron(torch.from_numpy(w1).to(CUDA), torch.from_numpy(w2).to(CUDA), 0.01,
                   torch.arange(rows, device=CUDA))  # fmt: skip
    more = (np.kron(w1, w2) * np.float32(0.01)).astype(np.float32)
    up = (rng.standard_normal((rows, rank)) * 0.02).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    seed = 1234
    if form == ob.NVFP4:
        codes, blocks = _nvfp4_stored(rows, cols, rng)
        want = ob.bake_nvfp4(codes, blocks, 0.03, up, down, seed, more=more)
        stored = {"weight": torch.from_numpy(codes).to(CUDA),
                  "scale": torch.from_numpy(blocks).view(torch.float8_e4m3fn).to(CUDA),
                  "scale_2": torch.tensor([0.03], device=CUDA)}  # fmt: skip
        cb.bake(torch, stored, _cuda(down), _cuda(up), seed=seed, more=cb.dense([kron]))
        assert np.array_equal(stored["scale"].view(torch.uint8).cpu().numpy(), want[1])
        assert np.array_equal(stored["weight"].cpu().numpy(), want[0])
        return
    data, scale, _ = _stored_for(form, rows, cols, 34)
    if form == ob.INT8:
        want = ob.bake(form, data, scale, up, ob.rotate_factor(down), seed, more=ob.rotate_factor(more))
        stored = {"weight": torch.from_numpy(data).to(CUDA), "scale": torch.from_numpy(scale).to(CUDA)}
        key = "weight"
    else:
        want = ob.bake(form, data, scale, up, down, seed, more=more)
        stored = {"value": _torch_data(form, data).to(CUDA)}
        key = "value"
    cb.bake(torch, stored, _cuda(down), _cuda(up), seed=seed, more=cb.dense([kron]))
    torch.cuda.synchronize()
    assert np.array_equal(_bytes(stored[key]), want.view(np.uint8).reshape(rows, -1))


def test_eager_entry_points_take_every_grid_option():
    """Every grid takes LoKr rows, a gain (nvfp4) and `Stats`: off the GPU each combination gets
    as far as the device check; an unknown grid or rounding is refused."""
    from cozyq import bake as cb

    t = torch.zeros(4, 16)
    down, up = torch.zeros(1, 16), torch.zeros(4, 1)
    dense = lambda a, b: torch.zeros(b - a, 16)  # noqa: E731
    with pytest.raises(ValueError, match="GPU"):
        cb.bake_rowwise(torch, t, torch.ones(4), down, up, 1.0)  # default grid "refit"
    with pytest.raises(ValueError, match="no grid"):
        cb.bake_rowwise(torch, t, torch.ones(4), down, up, 1.0, grid="wide")
    for grid in cb.GRIDS:
        with pytest.raises(ValueError, match="GPU"):
            cb.bake_rowwise(torch, t, torch.ones(4), down, up, 1.0, grid=grid, rounding="feedback", more=dense,
                            stats=cb.Stats())  # fmt: skip
        with pytest.raises(ValueError, match="GPU"):
            cb.bake_nvfp4(torch, t, t, torch.ones(1), down, up, 1.0, grid=grid, gain=torch.ones(4), more=dense,
                          seed=1, stats=cb.Stats())  # fmt: skip
    with pytest.raises(ValueError, match="GPU"):
        cb.bake_plain(torch, t, down, up, 1.0, stats=cb.Stats())  # Stats: built
    with pytest.raises(ValueError):
        cb.bake_int8_convrot(torch, t, t, down, up, 1.0, rounding="up")


def test_eager_noise_needs_a_seed_or_a_generator():
    """A stochastic eager bake takes `seed`, or draws a fresh 31-bit one from `generator` on
    each call; with neither it refuses instead of reusing one stream. Nearest needs none."""
    from cozyq import bake as cb

    t = torch.zeros(4, 16)
    down, up = torch.zeros(1, 16), torch.zeros(4, 1)
    with pytest.raises(ValueError, match="seed"):
        cb.bake_int8_convrot(torch, t, t, down, up, 1.0, rounding="stochastic")
    with pytest.raises(ValueError, match="seed"):
        cb.bake_nvfp4(torch, t, t, t, down, up, 1.0)
    gen = torch.Generator().manual_seed(5)
    drawn = [cb._noise_seed(torch, None, gen, True) for _ in range(4)]
    assert len(set(drawn)) == 4 and all(0 <= d <= cb.SEED_MASK for d in drawn)
    assert cb._noise_seed(torch, (1 << 40) + 7, None, True) == 7
    assert cb._noise_seed(torch, None, None, False) == 0


def test_kron_rows_against_torch_kron():
    """`Kron` rows against `torch.kron` (the library routine), whole and sliced, with an index
    that reorders and skips rows; `dense` sums terms and is None for none."""
    from cozyq import bake as cb

    gen = torch.Generator().manual_seed(9)
    w1, w2 = torch.randn(3, 4, generator=gen), torch.randn(5, 2, generator=gen)
    index = torch.tensor([14, 0, 7, 3, 9, 12])
    term = cb.Kron(w1, w2, 0.25, index)
    full = torch.kron(w1, w2) * 0.25
    assert torch.equal(term(0, 6), full[index])
    assert torch.equal(term(2, 5), full[index[2:5]])
    other = cb.Kron(w1 * 2, w2, 1.0, index)
    assert torch.allclose(cb.dense([term, other])(0, 6), full[index] + torch.kron(w1 * 2, w2)[index])
    assert cb.dense([]) is None


@pytest.mark.gpu
def test_gpu_eager_entry_points():
    """`bake_plain` / `bake_rowwise` / `bake_int8_convrot` / `bake_nvfp4` called directly, with
    alpha, as the reference's eager functions are: bit-exact against the oracle's laws."""
    from cozyq import bake as cb

    rng = np.random.default_rng(77)
    rows, cols, rank, alpha, seed = 40, 256, 4, 0.5, 99
    up = (rng.standard_normal((rows, rank)) * 0.04).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    up_a = (up * np.float32(alpha)).astype(np.float32)
    assert cb.serving(torch, 0) == "fused"
    # bf16 nearest with a gain
    data, _, _ = _stored_for(ob.BF16, rows, cols, 1)
    gain = (rng.random(rows) + 0.5).astype(np.float32)
    t = _torch_data(ob.BF16, data).to(CUDA)
    cb.bake_plain(torch, t, _cuda(down), _cuda(up), alpha, gain=_cuda(gain), seed=seed)
    assert np.array_equal(_bytes(t), ob.bake(ob.BF16, data, None, up_a, down, seed, gain=gain,
                                            nearest=True).view(np.uint8))  # fmt: skip
    # fp8.rowwise, keep, stochastic
    data, scale, _ = _stored_for(ob.ROWWISE, rows, cols, 2)
    w = torch.from_numpy(data).view(torch.float8_e4m3fn).to(CUDA)
    cb.bake_rowwise(torch, w, _cuda(scale), _cuda(down), _cuda(up), alpha, grid="keep", rounding="stochastic",
                    seed=seed)  # fmt: skip
    assert np.array_equal(w.view(torch.uint8).cpu().numpy(),
                          ob.bake(ob.ROWWISE, data, scale, up_a, down, seed, rescale=scale))  # the eager order
    # int8.convrot, nearest
    data, scale, _ = _stored_for(ob.INT8, rows, cols, 3)
    w = torch.from_numpy(data).to(CUDA)
    cb.bake_int8_convrot(torch, w, _cuda(scale), _cuda(down), _cuda(up), alpha, seed=seed)
    want = ob.bake(ob.INT8, data, scale, up_a, ob.rotate_factor(down), seed, nearest=True)
    assert np.array_equal(w.cpu().numpy(), want)
    # nvfp4, the eager law's roundings, stochastic
    codes, blocks = _nvfp4_stored(rows, cols, rng)
    c, b = torch.from_numpy(codes).to(CUDA), torch.from_numpy(blocks).view(torch.float8_e4m3fn).to(CUDA)
    cb.bake_nvfp4(torch, c, b, torch.tensor([0.03], device=CUDA), _cuda(down), _cuda(up), alpha, seed=seed)
    want = ob.bake_nvfp4(codes, blocks, 0.03, up_a, down, seed, gain=np.ones(rows, np.float32))
    assert np.array_equal(b.view(torch.uint8).cpu().numpy(), want[1])
    assert np.array_equal(c.cpu().numpy(), want[0])


def test_refit_scales_law():
    """`refit` puts each row's baked maximum at 448 exactly in payload units (before rounding);
    `regrid` lifts the scale by 1/32 to 3/32."""
    amax = np.float32([448.0, 0.0, 1.0, 1e-20, 3.5])
    refit = ob.refit_scales(amax, False)
    inv = np.float32(1 / 448)
    assert refit.tolist() == [np.float32(448) * inv, np.float32(1e-12), inv, np.float32(1e-12), np.float32(3.5) * inv]
    assert abs(float(refit[0]) - 1.0) <= 2**-23
    regrid = ob.refit_scales(amax, True)
    ratio = regrid.astype(np.float64) / refit
    assert ((ratio >= 1 + 1 / 32 - 1e-6) & (ratio <= 1 + 3 / 32 + 1e-6)).all()
    assert regrid[0] == np.float32(1.0) * np.float32(1 + 1 / 32)  # row 0: frac(0) = 0


@pytest.mark.gpu
@pytest.mark.parametrize("grid", ["refit", "regrid"])
@pytest.mark.parametrize("rounding", ["nearest", "stochastic"])
def test_gpu_bake_rowwise_new_grids(grid, rounding):
    """`bake_rowwise(grid=refit|regrid)`: the row maxima, the new scales and every code
    bit-exact against the oracle."""
    from cozyq import bake as cb

    rows, cols, rank, seed = 70, 300, 6, 321
    data, scale, rng = _stored_for(ob.ROWWISE, rows, cols, 60)
    up = (rng.standard_normal((rows, rank)) * 0.05).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    amax = ob.row_amax(data, scale, up, down)
    new = ob.refit_scales(amax, grid == "regrid")
    want = ob.bake(ob.ROWWISE, data, scale, up, down, seed, nearest=rounding == "nearest", rescale=new)
    w = torch.from_numpy(data).view(torch.float8_e4m3fn).to(CUDA)
    s = _cuda(scale)
    from cozyq import prebuilt

    got_amax = prebuilt.library(0).bake_norms(ob.ROWWISE, w.view(torch.uint8), s, _cuda(up), _cuda(down),
                                             cols=cols, amax=True)  # fmt: skip
    assert np.array_equal(got_amax.cpu().numpy(), amax)
    cb.bake_rowwise(torch, w, s, _cuda(down), _cuda(up), 1.0, rounding=rounding, grid=grid, seed=seed)
    torch.cuda.synchronize()
    assert np.array_equal(s.cpu().numpy().view(np.uint32), new.view(np.uint32))
    assert np.array_equal(w.view(torch.uint8).cpu().numpy(), want)


def test_feedback_known_run():
    """A run of 10.4s where E4M3's step is 1 (8..16): the carry cycles 0.4, -0.2, 0.2, -0.4, 0,
    so the codes repeat 10, 11, 10, 11, 10 and every five of them sum to 52 = 5 · 10.4; the
    34th column starts a new run (carry from zero)."""
    got = ob.e4m3_value(ob.e4m3_feedback(np.full((1, 34), 10.4, np.float32)))[0]
    assert got[:30].tolist() == [10, 11, 10, 11, 10] * 6
    assert got[32:].tolist() == [10, 11]
    neg = ob.e4m3_value(ob.e4m3_feedback(np.full((1, 5), -10.4, np.float32)))[0]
    assert neg.tolist() == [-10, -11, -10, -11, -10]


def test_feedback_keeps_run_sums():
    """Payloads already on the grid come back unchanged; off the grid, each run's stored sum
    stays within half a step (of the last element) of the payloads' sum, where rounding each
    element alone drifts by many steps on a biased run; ragged columns pad the last run."""
    grid = _e4m3_magnitudes()
    rng = np.random.default_rng(5)
    on = np.where(rng.random((9, 70)) < 0.5, -1, 1) * grid[rng.integers(0, 127, (9, 70))]
    on = on.astype(np.float32)
    assert np.array_equal(ob.e4m3_value(ob.e4m3_feedback(on)), on)
    payload = (rng.random((40, 200)) * 0.4 + 20.3).astype(np.float32)  # step 2 between 16 and 32
    fb = ob.e4m3_value(ob.e4m3_feedback(payload)).astype(np.float64)
    near = ob.e4m3_value(ob.e4m3_nearest(payload)).astype(np.float64)
    for start in range(0, 200, 32):
        stop = min(start + 32, 200)
        want = payload[:, start:stop].astype(np.float64).sum(1)
        assert (np.abs(fb[:, start:stop].sum(1) - want) <= 1.0 + 1e-3).all()
        if stop - start == 32:
            assert (np.abs(near[:, start:stop].sum(1) - want) > 8).all()
    sat = ob.e4m3_value(ob.e4m3_feedback(np.full((1, 3), 500.0, np.float32)))[0]
    assert sat.tolist() == [448, 448, 448]


def test_nvfp4_refit_is_saturation_free():
    """`refit`: the tensor's peak lands on 6 · 448 · level exactly as the reference sets it, no
    element's payload passes 6, and nearest rounding leaves each element within half a step
    (at most one unit) of its target; an all-zero tensor takes level 1 and stays zero."""
    rng = np.random.default_rng(8)
    rows, cols, rank = 24, 96, 5
    codes, blocks = _nvfp4_stored(rows, cols, rng)
    up = (rng.standard_normal((rows, rank)) * 0.3).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    new_codes, new_blocks, level = ob.bake_nvfp4_refit(codes, blocks, 0.05, up, down, 3, nearest=True)
    nib = np.stack((codes & 15, codes >> 4), axis=-1).reshape(rows, cols)
    scaled = (ob.e4m3_value(np.repeat(blocks, 16, axis=1)) * np.float32(0.05)).astype(np.float32)
    target = ((ob.e2m1_value(nib) * scaled).astype(np.float32) + ob.delta(up, down)).astype(np.float64)
    assert float(level) == np.float32(np.abs(target).max() / 2688.0)
    unit = np.repeat(ob.e4m3_value(new_blocks).astype(np.float64) * float(level), 16, axis=1)
    out = ob.e2m1_value(np.stack((new_codes & 15, new_codes >> 4), axis=-1).reshape(rows, cols)) * unit
    assert (np.abs(target) <= 6 * unit * (1 + 1e-6)).all()
    assert (np.abs(out - target) <= unit * (1 + 1e-6)).all()
    zero_codes, zero_blocks, one = ob.bake_nvfp4_refit(np.zeros_like(codes), blocks, 0.05,
                                                        np.zeros((rows, 0), np.float32),
                                                        np.zeros((0, cols), np.float32), 3)  # fmt: skip
    assert float(one) == 1.0 and not zero_blocks.any() and not (zero_codes & 0x77).any()


def test_stats_properties():
    from cozyq import bake as cb

    st = cb.Stats(layers=1, elements=10, weight_energy=100.0, delta_energy=4.0, error_energy=1.0, kept=3.0,
                  effect_energy=10.0, effect_error=0.1)  # fmt: skip
    assert st.retention == 0.75 and st.sqnr_db == 20.0 and abs(st.effect_snr_db - 20.0) < 1e-12
    other = cb.Stats(layers=2, elements=5, saturated=3)
    st.add(other)
    assert st.layers == 3 and st.elements == 15 and st.saturated == 3
    assert cb.Stats().retention == 1.0 and cb.Stats().sqnr_db == float("inf")
    assert set(st.document()) == {"layers", "elements", "retention", "sqnr_db", "effect_snr_db",
                                  "delta_to_weight_db", "saturated", "seconds"}  # fmt: skip


@pytest.mark.gpu
@pytest.mark.parametrize("rank", [5, 200])
@pytest.mark.parametrize("form", [ob.BF16, ob.F16, ob.F32, ob.ROWWISE, ob.INT8, ob.NVFP4])
def test_gpu_bake_stats_against_the_oracle(form, rank):
    """`bake(..., stats=Stats())`: the accounting kernel's sums against the oracle's `account`
    over the same weight before and after (float64 sums: to 1e-9; the rank-space energies, whose
    projections the kernel sums in float32, to 1e-4; the saturated count exactly). Rank 200
    takes the projections in two 128-rank slices."""
    from cozyq import bake as cb

    rng = np.random.default_rng(700 + form + rank)
    rows, cols, seed = 70, 256, 41
    big = 0.5 * math.sqrt(5 / rank)
    up = (rng.standard_normal((rows, rank)) * (big if form in (ob.ROWWISE, ob.INT8, ob.NVFP4) else 0.02)).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    stats = cb.Stats()
    if form == ob.NVFP4:
        codes, blocks = _nvfp4_stored(rows, cols, rng)
        stored = {"weight": torch.from_numpy(codes).to(CUDA),
                  "scale": torch.from_numpy(blocks).view(torch.float8_e4m3fn).to(CUDA),
                  "scale_2": torch.tensor([0.03], device=CUDA)}  # fmt: skip
        cb.bake(torch, stored, _cuda(down), _cuda(up), seed=seed, stats=stats)
        want = ob.account(form, codes, stored["weight"].cpu().numpy(), up, down, blocks_before=blocks,
                          blocks_after=stored["scale"].view(torch.uint8).cpu().numpy(), second=0.03)  # fmt: skip
    else:
        data, scale, _ = _stored_for(form, rows, cols, 701)
        if form in (ob.BF16, ob.F16, ob.F32):
            stored = {"value": _torch_data(form, data).to(CUDA)}
            key = "value"
        else:
            w = torch.from_numpy(data).to(CUDA)
            stored = {"weight": w.view(torch.float8_e4m3fn) if form == ob.ROWWISE else w, "scale": _cuda(scale)}
            key = "weight"
        cb.bake(torch, stored, _cuda(down), _cuda(up), seed=seed, stats=stats)
        after = _bytes(stored[key]).view(data.dtype).reshape(data.shape)
        used = ob.rotate_factor(down) if form == ob.INT8 else down
        want = ob.account(form, data, after, up, used, scale_before=scale, scale_after=scale)
    assert stats.layers == 1 and stats.elements == want["elements"] == rows * cols
    assert stats.saturated == want["saturated"]
    for name in ("weight_energy", "delta_energy", "error_energy", "kept"):
        assert abs(getattr(stats, name) - want[name]) <= 1e-9 * max(abs(want[name]), 1e-30) + 1e-30, name
    for name in ("effect_energy", "effect_error"):
        assert abs(getattr(stats, name) - want[name]) <= 1e-4 * abs(want[name]) + 1e-12, name
    if form in (ob.ROWWISE, ob.INT8):
        assert stats.saturated > 0  # the large delta drives kept-scale payloads past the grid



FEEDBACK_SHAPES = [(70, 300, 6), (129, 257, 33), (1, 1, 1), (64, 128, 0), (3, 40, 128)]


@pytest.mark.gpu
@pytest.mark.parametrize("grid", ["keep", "refit", "regrid"])
@pytest.mark.parametrize("rows,cols,rank", FEEDBACK_SHAPES)
def test_gpu_bake_rowwise_feedback(grid, rows, cols, rank):
    """`bake_rowwise(rounding="feedback")`: every code and new scale bit-exact against the oracle
    (`keep` with a delta large enough to saturate rows)."""
    from cozyq import bake as cb

    data, scale, rng = _stored_for(ob.ROWWISE, rows, cols, 61 + rank)
    up = (rng.standard_normal((rows, rank)) * (3.0 if grid == "keep" else 0.05)).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    new = scale if grid == "keep" else ob.refit_scales(ob.row_amax(data, scale, up, down), grid == "regrid")
    want = ob.bake_feedback(data, scale, up, down, new)
    w = torch.from_numpy(data).view(torch.float8_e4m3fn).to(CUDA)
    s = _cuda(scale)
    cb.bake_rowwise(torch, w, s, _cuda(down), _cuda(up), 1.0, rounding="feedback", grid=grid)
    torch.cuda.synchronize()
    assert np.array_equal(s.cpu().numpy().view(np.uint32), new.view(np.uint32))
    got = w.view(torch.uint8).cpu().numpy()
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} codes differ, first at {bad[0].tolist()}"


@pytest.mark.gpu
@pytest.mark.parametrize("nearest", [True, False])
@pytest.mark.parametrize("rows,cols,rank", [(40, 256, 4), (129, 272, 33), (1, 16, 1), (64, 128, 0)])
def test_gpu_bake_nvfp4_refit(nearest, rows, cols, rank):
    """`bake_nvfp4(grid="refit")`: the new second level, every block byte and every code
    bit-exact against the oracle (stochastic on the Philox stream)."""
    from cozyq import bake as cb

    rng = np.random.default_rng(rows + rank)
    codes, blocks = _nvfp4_stored(rows, cols, rng)
    up = (rng.standard_normal((rows, rank)) * 0.2).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    seed = 1234
    want_codes, want_blocks, level = ob.bake_nvfp4_refit(codes, blocks, 0.04, up, down, seed, nearest=nearest)
    c, b = torch.from_numpy(codes).to(CUDA), torch.from_numpy(blocks).view(torch.float8_e4m3fn).to(CUDA)
    second = torch.tensor([0.04], device=CUDA)
    cb.bake_nvfp4(torch, c, b, second, _cuda(down), _cuda(up), 1.0, grid="refit",
                  rounding="nearest" if nearest else "stochastic", seed=seed)  # fmt: skip
    torch.cuda.synchronize()
    assert second.cpu().numpy().view(np.uint32)[0] == np.float32(level).view(np.uint32)
    assert np.array_equal(b.view(torch.uint8).cpu().numpy(), want_blocks)
    assert np.array_equal(c.cpu().numpy(), want_codes)


@pytest.mark.gpu
def test_gpu_bake_nvfp4_refit_all_zero():
    """An all-zero nvfp4 weight with no delta refits to level 1 and zero blocks, as the
    reference's `amax > 0` test sets it."""
    from cozyq import bake as cb

    rows, cols = 8, 64
    c = torch.zeros(rows, cols // 2, dtype=torch.uint8, device=CUDA)
    b = torch.full((rows, cols // 16), 0x30, dtype=torch.uint8, device=CUDA).view(torch.float8_e4m3fn)
    second = torch.tensor([0.5], device=CUDA)
    cb.bake_nvfp4(torch, c, b, second, torch.zeros(0, cols, device=CUDA), torch.zeros(rows, 0, device=CUDA),
                  1.0, grid="refit", rounding="nearest")  # fmt: skip
    torch.cuda.synchronize()
    assert float(second) == 1.0
    assert not b.view(torch.uint8).any() and not c.any()


@pytest.mark.gpu
def test_gpu_torch_divides_by_a_python_float_as_a_reciprocal_multiply():
    """The eager bake's premise (`amax / (6.0 * second)`, `amax / 448`): torch on the GPU
    computes `tensor / python_float` as `tensor · float32(1 / float32(divisor))`, which differs
    from the IEEE quotient in the last bit for some inputs; the oracle's eager laws follow it."""
    rng = np.random.default_rng(3)
    a = (rng.random(1 << 16) * 100 + 1).astype(np.float32)
    for b in (448.0, 6.0 * 0.3, 6.0 * float(np.float32(0.07)), 2688.0):
        got = (torch.from_numpy(a).to(CUDA) / b).cpu().numpy()
        recip = (a * (np.float32(1) / np.float32(b))).astype(np.float32)
        assert np.array_equal(got.view(np.uint32), recip.view(np.uint32)), b
    assert not np.array_equal((a / np.float32(448.0)).astype(np.float32), (a * (np.float32(1) / np.float32(448.0))).astype(np.float32))


@pytest.mark.gpu
@pytest.mark.parametrize("rounding", ["nearest", "stochastic"])
def test_gpu_bake_rowwise_keep_eager_order(rounding):
    """`bake_rowwise(grid="keep")` with LoKr rows and `Stats`: codes `(decode · scale + delta) /
    scale` as the reference's eager bake orders them, the scale kept, bit-exact."""
    from cozyq import bake as cb

    rows, cols, rank, seed = 50, 200, 5, 77
    data, scale, rng = _stored_for(ob.ROWWISE, rows, cols, 62)
    up = (rng.standard_normal((rows, rank)) * 0.05).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    extra = (rng.standard_normal((rows, cols)) * 0.01).astype(np.float32)
    want = ob.bake(ob.ROWWISE, data, scale, up, down, seed, more=extra, nearest=rounding == "nearest",
                   rescale=scale)  # fmt: skip
    w = torch.from_numpy(data).view(torch.float8_e4m3fn).to(CUDA)
    s, dense = _cuda(scale), _cuda(extra)
    stats = cb.Stats()
    cb.bake_rowwise(torch, w, s, _cuda(down), _cuda(up), 1.0, rounding=rounding, grid="keep", seed=seed,
                    more=lambda a, b: dense[a:b], stats=stats)  # fmt: skip
    torch.cuda.synchronize()
    assert np.array_equal(s.cpu().numpy().view(np.uint32), scale.view(np.uint32))
    assert np.array_equal(w.view(torch.uint8).cpu().numpy(), want)
    assert stats.elements == rows * cols


def _exact_rank_one(rng, rows: int, cols: int):
    """A rank-one `u ⊗ v` whose float32 products are exact (few-bit integers times powers of
    two), so `fma(u, v, acc)` rounds exactly as `acc + (u · v)` does."""
    u = (rng.integers(-15, 16, rows) * 2.0 ** -6).astype(np.float32)
    v = (rng.integers(-15, 16, cols) * 2.0 ** -3).astype(np.float32)
    return u, v, np.outer(u, v).astype(np.float32)


def test_oracle_more_is_one_more_rank():
    """LoKr rows enter the delta after the chain: with `more = u ⊗ v` exact in float32, adding
    them equals the factors with `u`, `v` appended as the last rank (the chain's last FMA),
    for the rowwise row maxima, the feedback bake and the nvfp4 refit."""
    rng = np.random.default_rng(17)
    rows, cols, rank = 33, 96, 4
    data, scale, _ = _stored_for(ob.ROWWISE, rows, cols, 18)
    up = (rng.standard_normal((rows, rank)) * 0.05).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    u, v, more = _exact_rank_one(rng, rows, cols)
    up2, down2 = np.concatenate([up, u[:, None]], 1), np.concatenate([down, v[None, :]], 0)
    amax = ob.row_amax(data, scale, up, down, more)
    assert np.array_equal(amax, ob.row_amax(data, scale, up2, down2))
    assert not np.array_equal(amax, ob.row_amax(data, scale, up, down))
    new = ob.refit_scales(amax, False)
    assert np.array_equal(ob.bake_feedback(data, scale, up, down, new, more), ob.bake_feedback(data, scale, up2, down2, new))
    codes, blocks = _nvfp4_stored(rows, cols, rng)
    got = ob.bake_nvfp4_refit(codes, blocks, 0.05, up, down, 9, more=more)
    want = ob.bake_nvfp4_refit(codes, blocks, 0.05, up2, down2, 9)
    assert all(np.array_equal(a, b) for a, b in zip(got, want))


def test_oracle_refit_uniform_power_of_two_gain_is_a_level():
    """A gain of 2 on every row doubles each decoded value exactly, as decoding at twice the
    stored level does: the refit's codes, blocks and new level are the same either way; a
    per-row gain moves the level to the new peak."""
    rng = np.random.default_rng(19)
    rows, cols, rank = 20, 64, 3
    codes, blocks = _nvfp4_stored(rows, cols, rng)
    up = (rng.standard_normal((rows, rank)) * 0.1).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    two = np.full(rows, 2.0, np.float32)
    got = ob.bake_nvfp4_refit(codes, blocks, 0.03, up, down, 4, gain=two)
    want = ob.bake_nvfp4_refit(codes, blocks, 0.06, up, down, 4)
    assert all(np.array_equal(a, b) for a, b in zip(got, want))
    assert np.array_equal(ob.bake_nvfp4_refit(codes, blocks, 0.03, up, down, 4, gain=np.ones(rows, np.float32))[0],
                          ob.bake_nvfp4_refit(codes, blocks, 0.03, up, down, 4)[0])  # fmt: skip
    gain = np.linspace(0.5, 3.0, rows).astype(np.float32)
    _, _, level = ob.bake_nvfp4_refit(codes, blocks, 0.03, np.zeros((rows, 0), np.float32),
                                      np.zeros((0, cols), np.float32), 4, gain=gain)  # fmt: skip
    nib = np.stack((codes & 15, codes >> 4), axis=-1).reshape(rows, cols)
    scaled = (ob.e4m3_value(np.repeat(blocks.astype(np.int64), 16, axis=1)) * np.float32(0.03)).astype(np.float32)
    decoded = (ob.e2m1_value(nib) * scaled).astype(np.float32)
    peak = float(np.abs((decoded * gain[:, None]).astype(np.float32)).max())
    assert float(level) == np.float32(peak / 2688.0)


def test_oracle_account_decodes_after_at_the_new_level():
    """`account` with `second_after`: the error and kept energies against the weight decoded by
    the layout-law decoder (pinned by the reference's nvfp4 vectors) at each level. That decoder
    rounds `(e2m1 · scale) · level` once where the eager decode rounds `e2m1 · (scale · level)`
    twice, hence the 1e-4 tolerance; decoding after at the stale level misses by far more."""
    rng = np.random.default_rng(23)
    rows, cols, rank = 16, 64, 3
    codes, blocks = _nvfp4_stored(rows, cols, rng)
    up = (rng.standard_normal((rows, rank)) * 0.1).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    new_codes, new_blocks, level = ob.bake_nvfp4_refit(codes, blocks, 0.03, up, down, 4, nearest=True)
    got = ob.account(ob.NVFP4, codes, new_codes, up, down, blocks_before=blocks, blocks_after=new_blocks,
                     second=0.03, second_after=float(level))  # fmt: skip

    def decode(c, b, second):
        return laws.decode_nvfp4(torch.from_numpy(c), torch.from_numpy(b).view(torch.float8_e4m3fn),
                                 torch.tensor([second]), "row_major", False, False, None,
                                 torch.float32).double().numpy()  # fmt: skip

    base = decode(codes, blocks, 0.03)
    target = (base.astype(np.float32) + ob.delta(up, down)).astype(np.float32).astype(np.float64)
    stored = decode(new_codes, new_blocks, float(level))
    assert math.isclose(got["error_energy"], float(((stored - target) ** 2).sum()), rel_tol=1e-4)
    assert math.isclose(got["kept"], float(((stored - base) * ob.delta(up, down)).sum()), rel_tol=1e-4)
    assert got["saturated"] == 0  # refit is saturation-free
    stale = ob.account(ob.NVFP4, codes, new_codes, up, down, blocks_before=blocks, blocks_after=new_blocks,
                       second=0.03)  # fmt: skip
    assert not math.isclose(stale["error_energy"], got["error_energy"], rel_tol=1e-2)


@pytest.mark.gpu
@pytest.mark.parametrize("grid", ["refit", "regrid"])
@pytest.mark.parametrize("gain,more,nearest", [(True, False, True), (False, True, False), (True, True, False),
                                               (True, True, True)])
def test_gpu_bake_nvfp4_refit_options(grid, gain, more, nearest):
    """`bake_nvfp4(grid=refit|regrid)` with a DoRA gain, LoKr rows and `Stats`: the new level,
    every block byte and every code bit-exact against the oracle, the accounting against its
    `account` with the weight before at the stored level and after at the new one."""
    from cozyq import bake as cb

    rows, cols, rank, seed = 129, 272, 33, 555
    rng = np.random.default_rng(rows + int(gain) + 2 * int(more))
    codes, blocks = _nvfp4_stored(rows, cols, rng)
    up = (rng.standard_normal((rows, rank)) * 0.1).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    g = rng.uniform(0.5, 2.0, rows).astype(np.float32) if gain else None
    extra = (rng.standard_normal((rows, cols)) * 0.3).astype(np.float32) if more else None
    want_codes, want_blocks, level = ob.bake_nvfp4_refit(codes, blocks, 0.04, up, down, seed, nearest=nearest,
                                                         gain=g, more=extra)  # fmt: skip
    c, b = torch.from_numpy(codes).to(CUDA), torch.from_numpy(blocks).view(torch.float8_e4m3fn).to(CUDA)
    second = torch.tensor([0.04], device=CUDA)
    dense = _cuda(extra)
    stats = cb.Stats()
    cb.bake_nvfp4(torch, c, b, second, _cuda(down), _cuda(up), 1.0, grid=grid, seed=seed, stats=stats,
                  rounding="nearest" if nearest else "stochastic", gain=_cuda(g),
                  more=None if extra is None else (lambda a, z: dense[a:z]))  # fmt: skip
    torch.cuda.synchronize()
    assert second.cpu().numpy().view(np.uint32)[0] == np.float32(level).view(np.uint32)
    assert np.array_equal(b.view(torch.uint8).cpu().numpy(), want_blocks)
    assert np.array_equal(c.cpu().numpy(), want_codes)
    want = ob.account(ob.NVFP4, codes, want_codes, up, down, blocks_before=blocks, blocks_after=want_blocks,
                      second=0.04, second_after=float(level), gain=g, more=extra)  # fmt: skip
    assert stats.layers == 1 and stats.elements == rows * cols and stats.saturated == want["saturated"]
    for name in ("weight_energy", "delta_energy", "error_energy", "kept"):
        assert abs(getattr(stats, name) - want[name]) <= 1e-9 * max(abs(want[name]), 1e-30) + 1e-30, name
    for name in ("effect_energy", "effect_error"):
        assert abs(getattr(stats, name) - want[name]) <= 1e-4 * abs(want[name]) + 1e-12, name


@pytest.mark.gpu
@pytest.mark.parametrize("grid", ["keep", "refit", "regrid"])
@pytest.mark.parametrize("rounding", ["feedback", "nearest", "stochastic"])
def test_gpu_bake_rowwise_lokr_rows_on_every_grid(grid, rounding):
    """`bake_rowwise` with LoKr rows and `Stats` on every grid and rounding: the row maxima (with
    the rows), the new scales, every code and the accounting against the oracle."""
    from cozyq import bake as cb
    from cozyq import prebuilt

    rows, cols, rank, seed = 70, 300, 6, 99
    data, scale, rng = _stored_for(ob.ROWWISE, rows, cols, 64)
    up = (rng.standard_normal((rows, rank)) * 0.05).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    extra = (rng.standard_normal((rows, cols)) * 0.2).astype(np.float32)
    amax = ob.row_amax(data, scale, up, down, extra)
    new = scale if grid == "keep" else ob.refit_scales(amax, grid == "regrid")
    if rounding == "feedback":
        want = ob.bake_feedback(data, scale, up, down, new, extra)
    else:
        want = ob.bake(ob.ROWWISE, data, scale, up, down, seed, more=extra, nearest=rounding == "nearest",
                       rescale=new)  # fmt: skip
    w = torch.from_numpy(data).view(torch.float8_e4m3fn).to(CUDA)
    s, dense = _cuda(scale), _cuda(extra)
    got_amax = prebuilt.library(0).bake_norms(ob.ROWWISE, w.view(torch.uint8), s, _cuda(up), _cuda(down),
                                             cols=cols, amax=True, more=dense)  # fmt: skip
    assert np.array_equal(got_amax.cpu().numpy(), amax)
    stats = cb.Stats()
    cb.bake_rowwise(torch, w, s, _cuda(down), _cuda(up), 1.0, rounding=rounding, grid=grid, seed=seed,
                    more=lambda a, z: dense[a:z], stats=stats)  # fmt: skip
    torch.cuda.synchronize()
    assert np.array_equal(s.cpu().numpy().view(np.uint32), new.view(np.uint32))
    got = w.view(torch.uint8).cpu().numpy()
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} codes differ, first at {bad[0].tolist()}"
    acc = ob.account(ob.ROWWISE, data, want, up, down, scale_before=scale, scale_after=new, more=extra)
    assert stats.saturated == acc["saturated"] and stats.elements == rows * cols
    for name in ("weight_energy", "delta_energy", "error_energy", "kept"):
        assert abs(getattr(stats, name) - acc[name]) <= 1e-9 * max(abs(acc[name]), 1e-30) + 1e-30, name


@pytest.mark.gpu
def test_gpu_nvfp4_row_amax_with_gain_and_rows():
    """`cozyq_bake_row_amax` on nvfp4 with a gain and LoKr rows: each row's max of
    |gain · decode + up @ down + more| bit-exact against the oracle's target."""
    from cozyq import prebuilt

    rows, cols, rank = 65, 144, 7
    rng = np.random.default_rng(31)
    codes, blocks = _nvfp4_stored(rows, cols, rng)
    up = (rng.standard_normal((rows, rank)) * 0.1).astype(np.float32)
    down = rng.standard_normal((rank, cols)).astype(np.float32)
    g = rng.uniform(0.5, 2.0, rows).astype(np.float32)
    extra = (rng.standard_normal((rows, cols)) * 0.3).astype(np.float32)
    nib = np.stack((codes & 15, codes >> 4), axis=-1).reshape(rows, cols)
    scaled = (ob.e4m3_value(np.repeat(blocks.astype(np.int64), 16, axis=1)) * np.float32(0.04)).astype(np.float32)
    base = ((ob.e2m1_value(nib) * scaled).astype(np.float32) * g[:, None]).astype(np.float32)
    d = (ob.delta(up, down) + extra).astype(np.float32)
    want = np.abs((base + d).astype(np.float32)).max(axis=1)
    got = prebuilt.library(0).bake_norms(ob.NVFP4, torch.from_numpy(codes).to(CUDA), None, _cuda(up), _cuda(down),
                                        cols=cols, blocks=torch.from_numpy(blocks).to(CUDA),
                                        second=torch.tensor([0.04], device=CUDA), amax=True, gain=_cuda(g),
                                        more=_cuda(extra))  # fmt: skip
    assert np.array_equal(got.cpu().numpy(), want)

"""CPU restatement of the LoRA bake's fused law — TEST INFRASTRUCTURE ONLY (see `oracle/__init__`).

The reference bakes `up @ down` into a stored weight in place on the GPU with one Triton kernel
per stored form (`internal/lora_bake.py:775-815` `fused`, kernels `:955-1053`): bf16 (stochastic
by adding 16 noise bits), f16 and f32 (nearest), `fp8.rowwise` (E4M3 data, stochastic, row
scale kept), `int8-convrot256/1` (int8 of the rotated rows, stochastic floor, row scale kept,
`down` rotated by `rotate_factor`) and canonical `nvfp4` (E2M1 codes, E4M3 block scales kept
unless a block outgrows 7/6 of its scale, the f32 second level kept). The noise of element
(row, col) is Triton's Philox draw at counter `row * cols + col` (taken mod 2^32) under the
31-bit seed. Everything here is numpy float32 / uint32 arithmetic, operation for operation:

- `delta`: `up @ down` as one float32 FMA chain per element in rank order from +0 — the order an
  IEEE f32 `tl.dot`'s FMA lowering takes over `:1023-1033`. The FMA is exact (`fma32`).
- nvfp4's target is `fma(e2m1, scale·level, delta)`: the product-plus-delta at `:990` under
  Triton's default floating-point contraction. Every other mul/add of the kernels is separate.

Pins, exercised in `tests/test_bake.py`:
- `philox` (Philox4x32-10, Salmon et al., SC'11): the three published Random123 known-answer
  vectors (zero, all-ones and pi counters/keys).
- `randint`, `rand` (seed/offset mapping and the uint → [0, 1) map of Triton's `tl.randint` /
  `tl.rand`): `tests/golden/philox_vectors.json`, written by `tests/golden/make_philox_vectors.py`
  from Triton's own interpreter (the installed library, not the reference).
- `fma32`: exact rational arithmetic (`fractions.Fraction`) rounded to float32 by an
  independent integer rounding, over random and constructed near-tie triples.
- `e4m3_value`, `e4m3_stochastic`, `e4m3_at_least`, `e2m1_value`, `e2m1_stochastic`: brute force
  over every code and every neighbouring pair — exact grid values round to themselves under any
  noise, the result is always one of the two grid neighbours, rounding up happens exactly when
  the draw is under the covered fraction; `e4m3_at_least` is the least code whose value holds
  the need (against a sorted search of the 127 magnitudes).
- `bake`, `bake_nvfp4`: the reference's own self-check cases (`probe`, `:852-898`, exact
  results for every form over partial tiles and two inner steps); rank 0 writes back every byte
  (but the reserved E4M3 codes and signed zeros, as the law says); the mean over seeds of a
  stochastic bake is the exact target (statistical bound); nearest rounding for f16 against
  numpy's own cast.
- `bake_nvfp4_refit`: the saturation-free and half-step bounds of the refit grid, a uniform
  gain of 2 equal to decoding at twice the level, LoKr rows `u ⊗ v` (exact float32 products)
  equal to `u`, `v` appended as the chain's last rank (also for `row_amax`, `bake_feedback`);
  `e4m3_feedback` by a hand-worked run and run-sum conservation; `account`'s `second_after`
  against the layout-law decoder of `oracle/laws.py`.
- `rotate_factor`: the reference's Hadamard expression order (`internal/encoding/formats.py:
  664-671`, evaluated left to right, as `laws.hadamard`) and the closed form H·H = 256·I.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import laws

#: Stored forms (`internal/lora_bake.py:768`).
BF16, F16, F32, ROWWISE, INT8, NVFP4 = range(6)
#: A seed is 31 bits (`internal/lora_bake.py:770`).
SEED_MASK = 0x7FFFFFFF

# Philox4x32 constants: the Weyl key increments and the round multipliers.
_KEY_A, _KEY_B = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)
_ROUND_A, _ROUND_B = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
#: Triton's uint32 → [0, 1) scale, the largest float32 with (2^31 − 1)·scale < 1.
UNIFORM_SCALE = np.float32(4.6566127342e-10)

_F32 = np.float32
_U32 = np.uint32


# ----------------------------------------------------------------------------- noise


def philox(key: int, c0, c1=0, c2=0, c3=0, rounds: int = 10):
    """Philox4x32-`rounds` of counters (c0, c1, c2, c3) under the 64-bit key (lo, hi), uint32
    arrays. Each round: c0' = hi(B·c2) ^ c1 ^ k0, c2' = hi(A·c0) ^ c3 ^ k1, c1' = lo(B·c2),
    c3' = lo(A·c0), then the key adds its Weyl constants."""
    shape = np.broadcast(np.asarray(c0), np.asarray(c1), np.asarray(c2), np.asarray(c3)).shape
    c = [np.broadcast_to(np.asarray(v, dtype=np.uint64) & 0xFFFFFFFF, shape).astype(np.uint64)
         for v in (c0, c1, c2, c3)]  # fmt: skip
    k0, k1 = np.uint64(key & 0xFFFFFFFF), np.uint64((key >> 32) & 0xFFFFFFFF)
    mask = np.uint64(0xFFFFFFFF)
    for _ in range(rounds):
        pb, pa = _ROUND_B * c[2], _ROUND_A * c[0]
        c = [((pb >> np.uint64(32)) ^ c[1] ^ k0) & mask, pb & mask,
             ((pa >> np.uint64(32)) ^ c[3] ^ k1) & mask, pa & mask]  # fmt: skip
        k0 = (k0 + np.uint64(_KEY_A)) & mask
        k1 = (k1 + np.uint64(_KEY_B)) & mask
    return tuple(v.astype(np.uint32) for v in c)


def _key(seed: int) -> int:
    """Triton's key from an int32 seed argument: sign-extended to 64 bits (`tl.philox`)."""
    seed = int(seed) & 0xFFFFFFFF
    return seed | (0xFFFFFFFF << 32) if seed >= 1 << 31 else seed


def randint(seed: int, offset) -> np.ndarray:
    """`tl.randint(seed, offset)` for uint32 offsets: the first Philox output at counter
    (offset, 0, 0, 0)."""
    return philox(_key(seed), np.asarray(offset, dtype=np.uint64) & 0xFFFFFFFF)[0]


def rand(seed: int, offset) -> np.ndarray:
    """`tl.rand`: the int32 view of `randint` folded to non-negative (x < 0 → −x − 1), converted
    to float32 and times `UNIFORM_SCALE`; in [0, 1)."""
    x = randint(seed, offset).view(np.int32)
    folded = np.where(x < 0, ~x, x)
    return folded.astype(np.float32) * UNIFORM_SCALE


# ----------------------------------------------------------------------------- exact float32 FMA


def fma32(a, b, c) -> np.ndarray:
    """float32 fused multiply-add, correctly rounded: the float32 product is exact in float64,
    the float64 sum is made round-to-odd (TwoSum error, then the odd neighbour), and rounding a
    round-to-odd float64 to float32 is the correct rounding (Boldo & Melquiond, 2008)."""
    a64, b64, c64 = (np.asarray(v, dtype=np.float32).astype(np.float64) for v in (a, b, c))
    p = a64 * b64
    s = p + c64
    bb = s - p
    err = (p - (s - bb)) + (c64 - bb)
    bits = np.asarray(s).view(np.int64)
    even = (bits & 1) == 0
    away = (err > 0) == (s > 0)
    fix = (err != 0) & even & np.isfinite(s)
    bits = np.where(fix, bits + np.where(away, 1, -1), bits)
    return bits.view(np.float64).astype(np.float32)


def delta(up: np.ndarray, down: np.ndarray) -> np.ndarray:
    """`up @ down` (float32 `[rows, rank]` × `[rank, cols]`) as a float32 FMA chain per element
    over ranks 0, 1, ... from +0."""
    rows, rank = up.shape
    acc = np.zeros((rows, down.shape[1]), dtype=np.float32)
    for r in range(rank):
        acc = fma32(up[:, r : r + 1], down[r : r + 1, :], acc)
    return acc


# ----------------------------------------------------------------------------- grids


def e4m3_value(code) -> np.ndarray:
    """E4M3 bytes → float32, the two reserved codes saturating to ±448
    (`internal/lora_bake.py:901-909`)."""
    code = np.asarray(code).astype(np.int64)
    field, mantissa = (code >> 3) & 15, (code & 7).astype(np.float32)
    normal = (mantissa + _F32(8)) * ((field + 117) << 23).astype(np.uint32).view(np.float32)
    magnitude = np.where(field == 0, mantissa * _F32(0.001953125), normal).astype(np.float32)
    magnitude = np.where((code & 127) == 127, _F32(448), magnitude)
    return np.where(code > 127, -magnitude, magnitude).astype(np.float32)


def e4m3_stochastic(payload, noise) -> np.ndarray:
    """float32 payload → E4M3 byte, saturating at 448: twenty noise bits added under the three
    kept mantissa bits, the rest truncated; below 2^-6 the value is lifted by 2^-6 into the
    grid of step 2^-9 (`internal/lora_bake.py:911-922`). A NaN payload takes 448's code."""
    payload = np.asarray(payload, dtype=np.float32)
    magnitude = np.fmin(np.abs(payload), _F32(448))
    small = magnitude < _F32(0.015625)
    lifted = np.where(small, magnitude + _F32(0.015625), magnitude).astype(np.float32)
    kept = ((lifted.view(np.uint32) + (np.asarray(noise, dtype=np.uint32) >> 12)) >> 20).astype(np.int64)
    code = kept - np.where(small, 968, 960)
    return np.where(payload < 0, code | 128, code).astype(np.uint8)


def e4m3_at_least(need) -> np.ndarray:
    """The least E4M3 code (0..126) whose value holds `need` ≥ 0: its float32 bits rounded up
    to three mantissa bits, or below 2^-6 a count of 2^-9 (`internal/lora_bake.py:924-931`)."""
    need = np.asarray(need, dtype=np.float32)
    bits = ((need.view(np.uint32).astype(np.uint64) + 0xFFFFF) & 0xFFF00000).astype(np.int64)
    normal = (((bits >> 23) - 120) << 3) | ((bits >> 20) & 7)
    tiny = np.ceil(np.fmax(need * _F32(512), _F32(0))).astype(np.int64)
    code = np.where(need < _F32(0.015625), tiny, normal)
    return np.clip(code, 0, 126)


def e2m1_value(code) -> np.ndarray:
    """E2M1 codes (sign in bit 3) → float32 (`internal/lora_bake.py:933-940`)."""
    code = np.asarray(code).astype(np.int64)
    magnitude = np.asarray(laws.E2M1_VALUES[:8], dtype=np.float32)[code & 7]
    return np.where(code >= 8, -magnitude, magnitude).astype(np.float32)


def e2m1_stochastic(payload, draw) -> np.ndarray:
    """|payload| (block units, saturating at 6) → its E2M1 magnitude code, the upper neighbour
    when the draw is under the fraction of the step covered (`internal/lora_bake.py:942-953`)."""
    payload, draw = np.asarray(payload, dtype=np.float32), np.asarray(draw, dtype=np.float32)
    magnitude = np.fmin(np.abs(payload), _F32(6))
    step = np.where(magnitude < 2, _F32(0.5), np.where(magnitude < 4, _F32(1), _F32(2))).astype(np.float32)
    low = np.fmin(np.floor(magnitude / step) * step, _F32(6)).astype(np.float32)
    index = np.where(low < 2, low * 2, np.where(low < 4, low + 2, np.where(low < 6, 6, 7)))
    up = draw < ((magnitude - low) / step).astype(np.float32)
    return (index.astype(np.int64) + up).astype(np.int64)


# ----------------------------------------------------------------------------- bakes


def rotate_factor(down: np.ndarray) -> np.ndarray:
    """`down` `[rank, in]` in an `int8-convrot256/1` weight's basis: each 256 input channels
    times the unnormalized regular Hadamard in the reference's expression order, then 1/16
    (`internal/lora_bake.py:366-369`)."""
    rotated = laws.hadamard(torch.from_numpy(np.ascontiguousarray(down, dtype=np.float32)), 256)
    return rotated.numpy().astype(np.float32) * _F32(1.0 / 16)


def _offsets(rows: int, cols: int) -> np.ndarray:
    return (np.arange(rows, dtype=np.uint64)[:, None] * np.uint64(cols)
            + np.arange(cols, dtype=np.uint64)[None, :]) & np.uint64(0xFFFFFFFF)  # fmt: skip


def e4m3_nearest(payload) -> np.ndarray:
    """float32 payload → the nearest E4M3 byte, saturating at 448, ties to the even code, the
    sign bit for a negative payload only (`_nearest`, `internal/lora_bake.py:156-160`); the
    magnitude's code by torch's own round-to-nearest-even cast."""
    payload = np.asarray(payload, dtype=np.float32)
    magnitude = np.fmin(np.abs(payload), _F32(448))
    code = torch.from_numpy(np.ascontiguousarray(magnitude)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return np.where(payload < 0, code | 128, code).astype(np.uint8)


def e2m1_nearest(payload) -> np.ndarray:
    """|payload| → the nearest E2M1 magnitude code, ties to the even code, saturating at 6
    (`_e2m1` with `nearest`, `internal/lora_bake.py:435-455`), by a search of the eight
    magnitudes."""
    magnitude = np.fmin(np.abs(np.asarray(payload, dtype=np.float32)), _F32(6))
    grid = np.asarray(laws.E2M1_VALUES[:8], dtype=np.float32)
    low = np.clip(np.searchsorted(grid, magnitude, side="right") - 1, 0, 7)
    high = np.minimum(low + 1, 7)
    gap = grid[high] - grid[low]
    fraction = np.where(gap > 0, (magnitude - grid[low]) / np.where(gap > 0, gap, 1), 0).astype(np.float32)
    up = (fraction > 0.5) | ((fraction == 0.5) & (low % 2 == 1))
    return (low + up).astype(np.int64)


def _bf16_nearest(value: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(value, dtype=np.float32)).to(torch.bfloat16).view(
        torch.int16).numpy().view(np.uint16)  # fmt: skip


def bake(form: int, data: np.ndarray, scale: np.ndarray | None, up: np.ndarray, down: np.ndarray,
         seed: int, *, gain: np.ndarray | None = None, more: np.ndarray | None = None,
         nearest: bool = False, no_delta: bool = False,
         rescale: np.ndarray | None = None) -> np.ndarray:  # fmt: skip
    """The new stored data of one `_bake_kernel` form (`internal/lora_bake.py:1013-1053`):
    `data` `[rows, cols]` as stored (bf16 / f16 as uint16 bits, f32, E4M3 or int8 bytes),
    `scale` the float32 row scale of ROWWISE and INT8, `up` float32 `[rows, rank]`, `down`
    float32 `[rank, cols]` (INT8: already `rotate_factor`ed).

    The eager bake's additions (`bake_plain`, `bake_rowwise`, `bake_int8_convrot`,
    `gain_rows`, `:271-423,733-749`): `gain` float32 `[rows]` multiplies plain rows first,
    `more` float32 `[rows, cols]` adds to the delta, `nearest` rounds to nearest (ties to even)
    instead of stochastically, `no_delta` leaves the rows times their gain alone. Build law:
    the row-scaled forms keep the fused order `decode + delta / scale` under them too.
    `rescale` (ROWWISE, `bake_rowwise`'s `refit` / `regrid`, `:340-352`): each row's new scale;
    the payload is then the eager order `(decode · scale + delta) / new`."""
    rows, cols = data.shape
    d = delta(up.astype(np.float32), down.astype(np.float32))
    if more is not None:
        d = (d + more.astype(np.float32)).astype(np.float32)
    at = _offsets(rows, cols)
    if form == INT8:
        unit = scale.astype(np.float32).reshape(-1, 1)
        payload = data.astype(np.float32)
        if not no_delta:
            payload = (payload + (d / unit).astype(np.float32)).astype(np.float32)
        if nearest:
            stored = np.rint(payload)
        else:
            stored = np.floor((payload + rand(seed, at)).astype(np.float32))
        return np.clip(stored, -127, 127).astype(np.int8)
    if form == ROWWISE:
        unit = scale.astype(np.float32).reshape(-1, 1)
        payload = e4m3_value(data)
        if rescale is not None:
            target = ((payload * unit).astype(np.float32) + d).astype(np.float32)
            payload = (target / rescale.astype(np.float32).reshape(-1, 1)).astype(np.float32)
        elif not no_delta:
            payload = (payload + (d / unit).astype(np.float32)).astype(np.float32)
        return e4m3_nearest(payload) if nearest else e4m3_stochastic(payload, randint(seed, at))
    if form == BF16:
        value = (data.astype(np.uint32) << 16).view(np.float32)
    elif form == F16:
        value = data.view(np.float16).astype(np.float32)
    elif form == F32:
        value = data.astype(np.float32)
    else:
        raise ValueError(f"no bake form {form}")
    if gain is not None:
        value = (value * gain.astype(np.float32).reshape(-1, 1)).astype(np.float32)
    if not no_delta:
        value = (value + d).astype(np.float32)
    if form == BF16:
        if nearest:
            return _bf16_nearest(value)
        kept = (value.view(np.uint32) + (randint(seed, at) >> 16)) >> 16
        return kept.astype(np.uint16)
    if form == F16:
        return value.astype(np.float16).view(np.uint16)
    return value


def bake_nvfp4(data: np.ndarray, blocks: np.ndarray, second: float, up: np.ndarray,
               down: np.ndarray, seed: int, *, gain: np.ndarray | None = None,
               more: np.ndarray | None = None, nearest: bool = False,
               no_delta: bool = False) -> tuple[np.ndarray, np.ndarray]:  # fmt: skip
    """`_bake_nvfp4_kernel` (`internal/lora_bake.py:955-1011`): canonical nvfp4 codes `[rows,
    cols/2]` (element 2k in the low nibble) and E4M3 block bytes `[rows, cols/16]`, second level
    kept. A block's scale is kept unless its baked maximum needs more than 7/6 of it, then the
    least code that holds it; each element rounds stochastically on its block's grid and a zero
    keeps its stored sign. Returns the new (codes, blocks).

    With `gain`, `more`, `nearest` or `no_delta` (the eager `bake_nvfp4`, `:458-525`, and
    `gain_rows`): the target is `round(round(round(e2m1·(scale·level))·gain) + delta)`, each
    product and sum rounded, a block's need is its peak times the float32 reciprocal of
    `6·level` (torch's division by a Python scalar on the GPU), and `nearest` rounds E2M1 to
    nearest (ties to even)."""
    rows, cols = data.shape[0], 2 * data.shape[1]
    level = _F32(second)
    codes = np.stack((data & 15, data >> 4), axis=-1).reshape(rows, cols).astype(np.int64)
    scaled = np.repeat(blocks.astype(np.int64), 16, axis=1)
    d = delta(up.astype(np.float32), down.astype(np.float32))
    if more is not None:
        d = (d + more.astype(np.float32)).astype(np.float32)
    scale_level = (e4m3_value(scaled) * level).astype(np.float32)
    if gain is None and more is None and not nearest and not no_delta:
        target = fma32(e2m1_value(codes), scale_level, d)
    else:
        g = np.ones(rows, np.float32) if gain is None else gain.astype(np.float32)
        base = ((e2m1_value(codes) * scale_level).astype(np.float32) * g.reshape(-1, 1)).astype(np.float32)
        target = base if no_delta else (base + d).astype(np.float32)
    peak = np.abs(target).reshape(rows, -1, 16).max(axis=2)
    if gain is None and more is None and not nearest and not no_delta:
        need = (peak / (_F32(6) * level)).astype(np.float32)  # the Triton kernel: a division
    else:
        # The eager bake's `amax / (6.0 * second)` divides by a Python float: on the GPU, torch
        # multiplies by the float32 reciprocal of the float32 divisor.
        need = (peak * (_F32(1) / (_F32(6) * level)).astype(np.float32)).astype(np.float32)
    kept = blocks.astype(np.int64)
    grown = (need * _F32(6)).astype(np.float32) > (e4m3_value(kept) * _F32(7)).astype(np.float32)
    block = np.where(grown, e4m3_at_least(need), kept)
    unit = np.repeat((e4m3_value(block) * level).astype(np.float32), 16, axis=1)
    payload = (target / np.where(unit > 0, unit, _F32(1))).astype(np.float32)
    if nearest:
        nibble = e2m1_nearest(payload)
    else:
        nibble = e2m1_stochastic(payload, rand(seed, _offsets(rows, cols)))
    negative = np.where(target == 0, codes >= 8, target < 0)
    nibble = nibble | np.where(negative, 8, 0)
    packed = (nibble[:, 0::2] | (nibble[:, 1::2] << 4)).astype(np.uint8)
    return packed, block.astype(np.uint8)


def bake_nvfp4_refit(data: np.ndarray, blocks: np.ndarray, second: float, up: np.ndarray,
                     down: np.ndarray, seed: int, *, nearest: bool = False,
                     gain: np.ndarray | None = None, more: np.ndarray | None = None,
                     ) -> tuple[np.ndarray, np.ndarray, np.float32]:  # fmt: skip
    """`bake_nvfp4` with `grid="refit"` (`internal/lora_bake.py:495-525`): the eager target
    `round(round(e2m1·(scale·level))·gain) + round(delta + more)` (`decoded` then `_delta`,
    `:488-505`; no gain or `more`: those factors drop out); the new second level
    `amax / (6·448)` in float64 (a Python float there), 1 for an all-zero tensor; every block's
    scale the least E4M3 code at or above `peak / (6·second)` as torch divides by a Python
    scalar on its GPU (times the float32 reciprocal of the float32 divisor); the unit
    `e4m3(block) · float32(second)`, a payload of 0 where it is 0. Returns the new (codes,
    blocks, float32 second level)."""
    rows, cols = data.shape[0], 2 * data.shape[1]
    level = _F32(second)
    codes = np.stack((data & 15, data >> 4), axis=-1).reshape(rows, cols).astype(np.int64)
    scale_level = (e4m3_value(np.repeat(blocks.astype(np.int64), 16, axis=1)) * level).astype(np.float32)
    d = delta(up.astype(np.float32), down.astype(np.float32))
    if more is not None:
        d = (d + more.astype(np.float32)).astype(np.float32)
    base = (e2m1_value(codes) * scale_level).astype(np.float32)
    if gain is not None:
        base = (base * gain.astype(np.float32).reshape(-1, 1)).astype(np.float32)
    target = (base + d).astype(np.float32)
    amax = float(np.abs(target).max()) if target.size else 0.0
    new = amax / (448.0 * 6.0) if amax > 0 else 1.0
    new32 = _F32(new)
    inv = (_F32(1) / _F32(6.0 * new)).astype(np.float32)
    need = (np.abs(target).reshape(rows, -1, 16).max(axis=2) * inv).astype(np.float32)
    block = e4m3_at_least(need)
    unit = np.repeat((e4m3_value(block) * new32).astype(np.float32), 16, axis=1)
    payload = np.where(unit > 0, (target / np.where(unit > 0, unit, _F32(1))).astype(np.float32), _F32(0))
    if nearest:
        nibble = e2m1_nearest(payload)
    else:
        nibble = e2m1_stochastic(payload, rand(seed, _offsets(rows, cols)))
    negative = np.where(target == 0, codes >= 8, target < 0)
    nibble = nibble | np.where(negative, 8, 0)
    packed = (nibble[:, 0::2] | (nibble[:, 1::2] << 4)).astype(np.uint8)
    return packed, block.astype(np.uint8), new32


FEEDBACK_RUN = 32


def e4m3_feedback(payload: np.ndarray) -> np.ndarray:
    """`encode_e4m3` with `feedback` (`internal/lora_bake.py:163-197`): `[rows, cols]` float32
    payloads → E4M3 bytes, the columns padded with zeros to runs of 32; along each run the
    carried error (from +0) is added before `e4m3_nearest`, and the new carry is that sum minus
    the stored signed magnitude, all in float32."""
    payload = np.asarray(payload, dtype=np.float32)
    rows, cols = payload.shape
    pad = -cols % FEEDBACK_RUN
    runs = np.pad(payload, ((0, 0), (0, pad))).reshape(rows, -1, FEEDBACK_RUN)
    out = np.empty(runs.shape, dtype=np.uint8)
    carry = np.zeros(runs.shape[:2], dtype=np.float32)
    for k in range(FEEDBACK_RUN):
        want = (runs[..., k] + carry).astype(np.float32)
        code = e4m3_nearest(want)
        out[..., k] = code
        stored = e4m3_value(code & 0x7F)
        carry = (want - np.where(code >= 0x80, -stored, stored)).astype(np.float32)
    return out.reshape(rows, -1)[:, :cols]


def bake_feedback(data: np.ndarray, scale: np.ndarray, up: np.ndarray, down: np.ndarray,
                  fresh: np.ndarray, more: np.ndarray | None = None) -> np.ndarray:
    """`bake_rowwise` with `feedback` rounding (`internal/lora_bake.py:319-363`): payloads
    `(decode · scale + delta) / fresh` (`fresh` the row scales after the bake, `scale` itself for
    `keep`; delta `round(up @ down + more)` with LoKr rows) through `e4m3_feedback`."""
    d = delta(up.astype(np.float32), down.astype(np.float32))
    if more is not None:
        d = (d + more.astype(np.float32)).astype(np.float32)
    unit = scale.astype(np.float32).reshape(-1, 1)
    target = ((e4m3_value(data) * unit).astype(np.float32) + d).astype(np.float32)
    return e4m3_feedback((target / fresh.astype(np.float32).reshape(-1, 1)).astype(np.float32))


def row_amax(data: np.ndarray, scale: np.ndarray, up: np.ndarray, down: np.ndarray,
             more: np.ndarray | None = None) -> np.ndarray:
    """An fp8.rowwise weight's row maxima of |decode · scale + round(up @ down + more)|, float32
    — the amax `bake_rowwise`'s `refit` takes (`internal/lora_bake.py:344-346`)."""
    base = (e4m3_value(data) * scale.astype(np.float32).reshape(-1, 1)).astype(np.float32)
    d = delta(up.astype(np.float32), down.astype(np.float32))
    if more is not None:
        d = (d + more.astype(np.float32)).astype(np.float32)
    target = (base + d).astype(np.float32)
    return np.abs(target).max(axis=1).astype(np.float32)


def refit_scales(amax: np.ndarray, regrid: bool) -> np.ndarray:
    """`bake_rowwise`'s new row scales (`internal/lora_bake.py:344-349`), float32 operation for
    operation: `max(amax / 448, 1e-12)`, and for `regrid` times
    `1 + (1 + 2·frac(row · 0.6180339887)) / 32`. The reference runs these as torch ops on its GPU,
    where a tensor divided by a Python scalar is multiplied by the scalar's float32 reciprocal:
    `amax · RN(1/448)` (the /32 is exact either way)."""
    new = np.maximum((amax.astype(np.float32) * _F32(1.0 / 448.0)).astype(np.float32), _F32(1e-12))
    if regrid:
        row = np.arange(amax.shape[0], dtype=np.float32)
        x = (row * _F32(0.6180339887)).astype(np.float32)
        frac = (x - np.trunc(x)).astype(np.float32)
        factor = (_F32(1) + ((_F32(1) + (_F32(2) * frac).astype(np.float32)).astype(np.float32) / _F32(32))).astype(np.float32)
        new = (new * factor).astype(np.float32)
    return new.astype(np.float32)


def norms(form: int, data: np.ndarray, scale: np.ndarray | None, up: np.ndarray,
          down: np.ndarray, *, blocks: np.ndarray | None = None,
          second: float | None = None) -> np.ndarray:  # fmt: skip
    """`norms` (`internal/lora_bake.py:653-689`): each row's L2 norm of the decoded stored
    weight plus `up @ down` — decoded as the eager reference decodes (`value.float()`,
    `decode_e4m3(code)·scale`, `code·scale`, `e2m1·(e4m3(block)·level)`), the delta added in
    float32, the squares summed in float64. `form` NVFP4 takes codes `data` and `blocks`."""
    rows = data.shape[0]
    if form == NVFP4:
        cols = 2 * data.shape[1]
        codes = np.stack((data & 15, data >> 4), axis=-1).reshape(rows, cols)
        scaled = (e4m3_value(np.repeat(blocks.astype(np.int64), 16, axis=1)) * _F32(second)).astype(np.float32)
        value = (e2m1_value(codes) * scaled).astype(np.float32)
    elif form == BF16:
        value = (data.astype(np.uint32) << 16).view(np.float32)
    elif form == F16:
        value = data.view(np.float16).astype(np.float32)
    elif form == F32:
        value = data.astype(np.float32)
    elif form == ROWWISE:
        value = (e4m3_value(data) * scale.astype(np.float32).reshape(-1, 1)).astype(np.float32)
    else:
        value = (data.astype(np.float32) * scale.astype(np.float32).reshape(-1, 1)).astype(np.float32)
    target = (value + delta(up.astype(np.float32), down.astype(np.float32))).astype(np.float64)
    return np.sqrt((target * target).sum(axis=1)).astype(np.float32)


def account(form: int, before: np.ndarray, after: np.ndarray, up: np.ndarray, down: np.ndarray, *,
            scale_before: np.ndarray | None = None, scale_after: np.ndarray | None = None,
            blocks_before: np.ndarray | None = None, blocks_after: np.ndarray | None = None,
            second: float = 1.0, second_after: float | None = None, gain: np.ndarray | None = None,
            more: np.ndarray | None = None) -> dict[str, float]:  # fmt: skip
    """`_account` (`internal/lora_bake.py:249-268`) of one bake from the weight before and after:
    base and stored decoded as the eager reference decodes, delta the FMA chain (plus `more`),
    target = base + delta in float32, the sums in float64; saturation by each form's payload
    (`|target / scale| > 464`, `|code + delta / scale| > 127.5`, `|target / unit| > 6`). nvfp4's
    `before` decodes at `second`, its `after` at `second_after` (a `refit`'s new level; `second`
    when None)."""
    level_after = second if second_after is None else second_after

    def decoded(data, scale, blocks, level=second):
        if form == NVFP4:
            rows, cols = data.shape[0], 2 * data.shape[1]
            codes = np.stack((data & 15, data >> 4), axis=-1).reshape(rows, cols)
            s = (e4m3_value(np.repeat(blocks.astype(np.int64), 16, axis=1)) * _F32(level)).astype(np.float32)
            return (e2m1_value(codes) * s).astype(np.float32)
        if form == BF16:
            return (data.astype(np.uint32) << 16).view(np.float32)
        if form == F16:
            return data.view(np.float16).astype(np.float32)
        if form == F32:
            return data.astype(np.float32)
        if form == ROWWISE:
            return (e4m3_value(data) * scale.astype(np.float32).reshape(-1, 1)).astype(np.float32)
        return (data.astype(np.float32) * scale.astype(np.float32).reshape(-1, 1)).astype(np.float32)

    base = decoded(before, scale_before, blocks_before)
    if gain is not None and form in (BF16, F16, F32, NVFP4):
        base = (base * gain.astype(np.float32).reshape(-1, 1)).astype(np.float32)
    d = delta(up.astype(np.float32), down.astype(np.float32))
    if more is not None:
        d = (d + more.astype(np.float32)).astype(np.float32)
    target = (base + d).astype(np.float32)
    stored = decoded(after, scale_after, blocks_after, level_after)
    err = (stored - target).astype(np.float32)
    if form == ROWWISE:
        saturated = int((np.abs((target / scale_after.astype(np.float32).reshape(-1, 1)).astype(np.float32)) > 464).sum())
    elif form == INT8:
        payload = (before.astype(np.float32) + (d / scale_before.astype(np.float32).reshape(-1, 1)).astype(np.float32))
        saturated = int((np.abs(payload.astype(np.float32)) > 127.5).sum())
    elif form == NVFP4:
        unit = np.repeat((e4m3_value(blocks_after.astype(np.int64)) * _F32(level_after)).astype(np.float32), 16, axis=1)
        ratio = (target / np.where(unit > 0, unit, _F32(1))).astype(np.float32)
        saturated = int(((unit > 0) & (np.abs(ratio) > 6)).sum())
    else:
        saturated = 0
    basis = down.astype(np.float64).T
    d64, e64 = d.astype(np.float64), err.astype(np.float64)
    return {
        "weight_energy": float((target.astype(np.float64) ** 2).sum()),
        "delta_energy": float((d64 ** 2).sum()),
        "error_energy": float((e64 ** 2).sum()),
        "kept": float(((stored.astype(np.float64) - base.astype(np.float64)) * d64).sum()),
        "saturated": saturated,
        "effect_energy": float(((d64 @ basis) ** 2).sum()),
        "effect_error": float(((e64 @ basis) ** 2).sum()),
        "elements": int(target.size),
    }

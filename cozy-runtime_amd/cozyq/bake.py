"""The LoRA bake on gfx950, under the names of cozy-runtime's `internal/lora_bake.py`.

A LoRA's `up @ down` is added into a stored weight in place and rounded back onto the weight's
own form, so the adapted layer serves at the speed of the unadapted one. The surface —
`bakeable`, `rotate_factor`, `fused`, `bake`, `probe`, `recipe`, the eager entry points and the
form constants — runs on the kernels of `csrc/bake.hip`.

The fused bake (`fused`, `bake`) covers:
- plain bf16 (stochastic: 16 noise bits under the kept ones), f16 and f32 (nearest);
- fp8.rowwise (E4M3 data, stochastic, row scale kept);
- int8.convrot (stochastic floor, row scale kept, `down` rotated into the weight's basis);
- canonical nvfp4 (E2M1 on the kept block grid; a block's E4M3 scale refitted only past 7/6 of
  it; the second level kept).
Element (row, col) draws Triton's Philox word at counter `row · cols + col` under the 31-bit
seed. The delta is one float32 FMA chain in rank order. The bytes equal `oracle/bake.py`'s.
Byte parity with the reference's Triton bake rests on reading its `tl.dot` as that chain.

The eager options run on the same kernels:
- a DoRA gain;
- LoKr rows (`more`, `Kron`, `dense`);
- `gain_rows`, `norms` and the `dora` helpers;
- `bake_rowwise`'s `keep` / `refit` / `regrid` grids and its error-feedback rounding;
- nvfp4's `refit` grid;
- `Stats` (any rank).
`alpha` scales `up` before the product. The reference scales the product after it, which gives
the same bytes when alpha is a power of two and can differ in the last bit otherwise.
A stochastic eager bake takes its noise from `seed` or draws `seed` from `generator`; without
either it refuses, rather than reuse one stream.

Every grid takes a gain (plain and nvfp4 forms), LoKr rows and `Stats`; nvfp4's `regrid` is
its `refit`, as in the reference (`grid != "keep"`). Tensors off the GPU raise ValueError.
"""

from __future__ import annotations

import math
import time
from collections.abc import Callable, Mapping, Sequence
from dataclasses import dataclass
from typing import Any, NamedTuple

Tensor = Any

#: Names the bytes a bake writes (`internal/lora_bake.py:58`).
VARIANT = "cozy.lora-bake/2"
#: Stored forms (`internal/lora_bake.py:768`), the first five as `cozyq_bake`'s `form`.
BF16, F16, F32, ROWWISE, INT8, NVFP4 = range(6)
#: A seed is 31 bits (`internal/lora_bake.py:770`).
SEED_MASK = 0x7FFFFFFF
#: The canonical stored nvfp4 a bake writes (`internal/lora_bake.py:412-417`).
NVFP4_PARAMS = {
    "block_size": 16,
    "global_scale": "multiply",
    "nibble_order": "low_first",
    "scale_layout": "row_major",
}
#: The rotation a baked int8.convrot weight carries (`int8-convrot256/1`).
CONVROT_GROUP = 256
#: `cozyq_bake`'s flags: round to nearest instead of stochastically; the rows times their gain
#: alone.
NEAREST, NO_DELTA = 1, 2
#: A dense delta's rows `[start, stop)`, float32 `[rows, in]`, added beside `up @ down`
#: (`internal/lora_bake.py:207`).
Dense = Callable[[int, int], Tensor]


class Verdict(NamedTuple):
    ok: bool
    detail: str


#: `Stats`' running sums, in the order of the accounting kernel's partials where they come
#: from it.
_SUMS = ("layers", "elements", "weight_energy", "delta_energy", "error_energy", "kept",
         "effect_energy", "effect_error", "saturated", "seconds")  # fmt: skip


@dataclass(slots=True)
class Stats:
    """Accumulated accounting of one or more bakes (rule B2; the reference's `Stats`,
    `internal/lora_bake.py:78-123`). Energies are sums of squares in the weight's own units:
    of the baked target W + delta (`weight_energy`), of the delta, and of the rounding error
    stored − target. `kept` is the inner product of what changed in storage with the delta.
    `effect_*` project the delta and the error onto the LoRA's own input directions
    (`· downᵀ`). `saturated` counts elements clipped at the grid's edge."""

    layers: int = 0
    elements: int = 0
    weight_energy: float = 0.0
    delta_energy: float = 0.0
    error_energy: float = 0.0
    kept: float = 0.0
    effect_energy: float = 0.0
    effect_error: float = 0.0
    saturated: int = 0
    seconds: float = 0.0

    @property
    def retention(self) -> float:
        """Fraction of the delta's own direction that reached storage (1.0 when there was no
        delta)."""
        if not self.delta_energy:
            return 1.0
        return self.kept / self.delta_energy

    @property
    def sqnr_db(self) -> float:
        """Target energy over rounding-error energy, in dB."""
        return _ratio_db(self.weight_energy, self.error_energy)

    @property
    def effect_snr_db(self) -> float:
        """The delta's effect on its own inputs over the error's, in dB."""
        return _ratio_db(self.effect_energy, self.effect_error)

    def add(self, other: Stats) -> None:
        for name in _SUMS:
            setattr(self, name, getattr(self, name) + getattr(other, name))

    def document(self) -> dict[str, float | int]:
        figures: dict[str, float | int] = {"layers": self.layers, "elements": self.elements}
        figures.update(retention=self.retention, sqnr_db=self.sqnr_db, effect_snr_db=self.effect_snr_db,
                       delta_to_weight_db=_ratio_db(self.delta_energy, self.weight_energy))  # fmt: skip
        figures.update(saturated=self.saturated, seconds=self.seconds)
        return figures


def _ratio_db(signal: float, noise: float) -> float:
    """10·log10(signal / noise): +inf without noise, -inf without signal."""
    if noise <= 0:
        return math.inf
    if signal <= 0:
        return -math.inf
    return 10 * math.log10(signal / noise)


def _account(torch: Any, stats: Stats, form: int, before: dict[str, Tensor], after: dict[str, Tensor],
             up: Tensor, down: Tensor, cols: int, gain: Tensor | None, more: Tensor | None,
             began: float) -> None:  # fmt: skip
    """One bake's sums into `stats` (`_account` and `_finish`, `internal/lora_bake.py:249-268,
    528-534`): `cozyq_bake_stats`' per-group partials, added in group order on the host."""
    data = after["data"]
    partial = _ops(data).bake_stats(form, before, after, up, down, cols=cols, gain=gain, more=more)
    sums = partial.cpu().sum(0).tolist()
    stats.weight_energy += sums[0]
    stats.delta_energy += sums[1]
    stats.error_energy += sums[2]
    stats.kept += sums[3]
    stats.saturated += int(round(sums[4]))
    stats.effect_energy += sums[5]
    stats.effect_error += sums[6]
    stats.elements += int(data.shape[0]) * cols
    torch.cuda.synchronize(data.device)
    stats.layers += 1
    stats.seconds += time.perf_counter() - began


#: Role signatures (role -> stored dtype) a bake takes, per scheme (rule B1).
_BAKEABLE_ROLES: dict[str, tuple[dict[str, str], ...]] = {
    "plain": ({"value": "bf16"}, {"value": "f16"}, {"value": "f32"}),
    "fp8.rowwise": ({"weight": "f8_e4m3fn", "scale": "f32"},),
    "int8.convrot": ({"weight": "i8", "scale": "f32"},),
    "nvfp4": ({"weight": "u8", "scale": "f8_e4m3fn", "scale_2": "f32"},),
}
#: Roles a scheme may carry that are not the weight's and stay out of the signature.
_IGNORED_ROLES = {"nvfp4": frozenset({"input_scale"})}


def bakeable(scheme: str, params: Mapping[str, object], roles: Mapping[str, str]) -> bool:
    """Whether a stored weight, given as scheme, params and role -> dtype, takes `bake` (rule
    B1; the reference's `bakeable`, `internal/lora_bake.py:537-551`). The scheme decides, not
    the roles: int8.rowwise stores what int8.convrot stores and is not rotated. Here an
    int8.convrot weight must also carry the 256 rotation that `down` is rotated by."""
    signatures = _BAKEABLE_ROLES.get(scheme)
    if signatures is None:
        return False
    ignored = _IGNORED_ROLES.get(scheme, frozenset())
    if {r: d for r, d in roles.items() if r not in ignored} not in signatures:
        return False
    if scheme == "nvfp4":
        return all(params.get(name, wanted) == wanted for name, wanted in NVFP4_PARAMS.items())
    if scheme == "int8.convrot":
        return int(params.get("rotation_size", CONVROT_GROUP)) == CONVROT_GROUP  # type: ignore[call-overload]
    return True


def _ops(tensor: Tensor):
    from cozyq import prebuilt

    if not tensor.is_cuda:
        raise ValueError("cozyq bakes on the GPU: the stored weight is not on a cuda device")
    return prebuilt.library(tensor.get_device())


def rotate_factor(torch: Any, down: Tensor) -> Tensor:
    """`down` (`[rank, in]`) in an `int8-convrot256/1` weight's basis
    (`internal/lora_bake.py:366-369`): each 256 input channels times the regular Hadamard / 16,
    float32."""
    return _ops(down).rotate_factor(down.to(torch.float32).contiguous())


@dataclass(frozen=True, slots=True)
class Kron:
    """A LoKr term (rule B3; `internal/lora_bake.py:210-224`): `scale · kron(w1, w2)` for
    `w1` `[a, b]` and `w2` `[c, d]`, restricted to the product rows `index` (int64, in order).
    Called with `(start, stop)` it gives rows `index[start:stop]`, float32 `[n, b·d]`."""

    w1: Tensor
    w2: Tensor
    scale: float
    index: Tensor

    def __call__(self, start: int, stop: int) -> Tensor:
        rows = self.index[start:stop]
        c = self.w2.shape[0]
        outer, inner = rows.div(c, rounding_mode="floor"), rows.remainder(c)  # row = outer · c + inner
        left = self.w1.index_select(0, outer).float()
        right = self.w2.index_select(0, inner).float()
        block = left.unsqueeze(2) * right.unsqueeze(1)  # [n, b, d]: w1[p, i] · w2[q, j]
        return block.reshape(block.shape[0], -1).mul_(self.scale)


class _DenseSum:
    """Rows of the sum of several LoKr terms, the first term's rows accumulated in place."""

    __slots__ = ("terms",)

    def __init__(self, terms: Sequence[Kron]) -> None:
        self.terms = tuple(terms)

    def __call__(self, start: int, stop: int) -> Tensor:
        total = self.terms[0](start, stop)
        for term in self.terms[1:]:
            total.add_(term(start, stop))
        return total


def dense(terms: Sequence[Kron]) -> Dense | None:
    """The dense rows of `terms` summed, or None for no terms (`internal/lora_bake.py:227-239`)."""
    return _DenseSum(terms) if terms else None


def _more_rows(torch: Any, more: Dense | None, rows: int, rotated: bool) -> Tensor | None:
    if more is None:
        return None
    block = more(0, rows).to(torch.float32).contiguous()
    return rotate_factor(torch, block) if rotated else block


def fused(torch: Any, stored: dict[str, Tensor], down: Tensor, up: Tensor, seed: int, *,
          gain: Tensor | None = None, more: Dense | None = None, flags: int = 0,
          stats: Stats | None = None) -> None:  # fmt: skip
    """`bake`, one kernel launch (`internal/lora_bake.py:775-815`): each tile adds its
    `up @ down` (float32) to the decoded stored values and rounds them back in place. `gain`
    (plain and nvfp4 rows), `more` and `flags` are the eager bake's additions; `stats` takes the
    bake's accounting from a copy of the weight before it."""
    began = time.perf_counter()
    up32 = up.to(torch.float32).contiguous()
    down32 = down.to(torch.float32).contiguous()
    gain32 = None if gain is None else gain.to(torch.float32).reshape(-1).contiguous()
    if "scale_2" in stored:
        raw = stored["weight"].view(torch.uint8)
        blocks = stored["scale"].view(torch.uint8)
        second = stored["scale_2"].to(torch.float32).reshape(1)
        rows = raw.shape[0]
        more_rows = _more_rows(torch, more, rows, False)
        before = None if stats is None else {"data": raw.clone(), "blocks": blocks.clone(), "second": second}
        _ops(raw).bake_nvfp4(raw, blocks, second, up32, down32, seed & SEED_MASK, gain=gain32,
                             more=more_rows, flags=flags)  # fmt: skip
        if stats is not None:
            after = {"data": raw, "blocks": blocks, "second": second}
            _account(torch, stats, NVFP4, before, after, up32, down32, 2 * raw.shape[1], gain32, more_rows, began)
        return
    rotated = False
    if "value" in stored:
        data = stored["value"]
        kinds = {torch.bfloat16: BF16, torch.float16: F16, torch.float32: F32}
        if data.dtype not in kinds:
            raise ValueError(f"a plain bake stores bf16, f16 or f32, not {data.dtype}")
        kind, scale = kinds[data.dtype], None
    elif stored["weight"].dtype == torch.int8:
        data, scale, kind = stored["weight"], stored["scale"].reshape(-1), INT8
        down32, rotated = rotate_factor(torch, down32), True
    else:
        data, scale, kind = stored["weight"].view(torch.uint8), stored["scale"].reshape(-1), ROWWISE
    if scale is not None and (scale.dtype != torch.float32 or not scale.is_contiguous()):
        raise ValueError("a row-scaled bake keeps a contiguous float32 row scale")
    if scale is not None and gain32 is not None:
        raise ValueError("a row-scaled weight takes its gain in its scale")
    more_rows = _more_rows(torch, more, data.shape[0], rotated)
    before = None
    if stats is not None:
        before = {"data": data.clone()} if scale is None else {"data": data.clone(), "scale": scale}
    _ops(data).bake(kind, data, scale, up32, down32, seed & SEED_MASK, gain=gain32, more=more_rows,
                    flags=flags)  # fmt: skip
    if stats is not None:
        after = {"data": data} if scale is None else {"data": data, "scale": scale}
        _account(torch, stats, kind, before, after, up32, down32, data.shape[1], gain32, more_rows, began)


def bake(
    torch: Any,
    stored: dict[str, Tensor],
    down: Tensor,
    up: Tensor,
    *,
    seed: int,
    stats: Any = None,
    how: str | None = "fused",
    gain: Tensor | None = None,
    more: Dense | None = None,
) -> None:
    """Bake `up @ down` into one stored weight by its roles (`internal/lora_bake.py:554-645`):
    plain floats, `fp8.rowwise`, `int8-convrot256/1` or canonical `nvfp4`. bf16, E4M3, int8 and
    E2M1 round stochastically, scales kept; `seed` names the weight's noise. A convolution's
    weight and factors bake as matrices, each kernel tap one more input column. `gain` (float32
    per output row, a DoRA's) scales the stored rows first: a row-scaled weight's scale exactly, a
    plain or nvfp4 one's values, rounded once with the delta. `more` (a LoKr's dense rows,
    `dense`) adds beside `up @ down`. `how` is accepted for the reference's callers: every bake
    runs on the HIP kernels. `down` and `up` may have rank 0."""
    if down.dim() > 2:
        stored = {role: t.view(t.shape[0], -1) if t.dim() > 2 else t for role, t in stored.items()}
        down, up = down.flatten(1), up.flatten(1)
    if gain is not None and "value" not in stored and "scale_2" not in stored:
        stored["scale"].view(-1).mul_(gain)
        gain = None
    if how not in ("fused", "eager", None):
        raise ValueError(f"no bake path {how!r}")
    fused(torch, stored, down, up, seed, gain=gain, more=more, stats=stats)


ROUNDINGS = ("nearest", "stochastic", "feedback")
GRIDS = ("keep", "refit", "regrid")


def _rounding_flags(rounding: str, allowed: tuple[str, ...] = ("nearest", "stochastic")) -> int:
    if rounding not in ROUNDINGS:
        raise ValueError(f"no rounding {rounding!r}")
    if rounding not in allowed:
        raise NotImplementedError(f"cozyq bakes by nearest or stochastic rounding, not {rounding!r}")
    return NEAREST if rounding == "nearest" else 0


def _noise_seed(torch: Any, seed: int | None, generator: Any, stochastic: bool) -> int:
    """The 31-bit seed of an eager bake's noise: `seed` when given, else one drawn from
    `generator` (so successive bakes from one generator get fresh streams, as the reference's
    torch draws do). A stochastic bake with neither raises; a nearest one needs no noise."""
    if seed is not None:
        return int(seed) & SEED_MASK
    if generator is not None:
        return int(torch.randint(0, SEED_MASK + 1, (1,), generator=generator, device=generator.device).item())
    if stochastic:
        raise ValueError("a stochastic bake draws its noise from `seed` or `generator`; give one")
    return 0


def _scaled_up(torch: Any, up: Tensor, alpha: float) -> Tensor:
    """`up` times `alpha` before the product: the reference scales the product instead
    (`_delta`, `internal/lora_bake.py:242-246`), the same for a power of two and within a float32
    rounding otherwise. `bake` itself always passes 1."""
    up32 = up.to(torch.float32)
    return up32 if alpha == 1.0 else up32 * alpha


def bake_plain(torch: Any, weight: Tensor, down: Tensor, up: Tensor, alpha: float, *,
               rounding: str = "nearest", generator: Any = None, stats: Any = None,
               more: Dense | None = None, gain: Tensor | None = None, seed: int | None = None) -> None:  # fmt: skip
    """`weight = gain * weight + alpha * up @ down`, float32, rounded once to its dtype
    (`internal/lora_bake.py:271-305`); bf16 rounds stochastically on request, other dtypes to
    nearest. The noise is the Philox stream under `seed`, or under a seed drawn from
    `generator`."""
    flags = _rounding_flags(rounding)
    if weight.dtype != torch.bfloat16:
        flags = NEAREST
    seed = _noise_seed(torch, seed, generator, flags == 0)
    fused(torch, {"value": weight}, down, _scaled_up(torch, up, alpha), seed, gain=gain, more=more,
          flags=flags, stats=stats)  # fmt: skip


#: `bake_rowwise`'s floor of a refitted row scale and E4M3's largest value
#: (`internal/lora_bake.py:72`, `internal/encoding/formats.py:497`).
ROW_SCALE_FLOOR, E4M3_MAX = 1e-12, 448.0


def bake_rowwise(torch: Any, data: Tensor, scale: Tensor, down: Tensor, up: Tensor, alpha: float, *,
                 rounding: str = "nearest", grid: str = "refit", generator: Any = None,
                 stats: Any = None, more: Dense | None = None, seed: int | None = None) -> None:  # fmt: skip
    """Bake into `fp8.rowwise` (`internal/lora_bake.py:319-363`): `data` `[out, in]` E4M3,
    `scale` one float32 per output row. `keep` rounds on the stored grid; `refit` sets each row's scale from its baked maximum,
    `max(amax / 448, 1e-12)`, and `regrid` raises that by 1/32 to 3/32 by the row's golden-ratio
    fraction, so every element rounds afresh. On every grid the codes are
    `(decode · scale + delta) / new` (`new` the kept scale for `keep`), the eager law's order,
    and `scale` takes the new values. `feedback` rounding (any grid) rounds
    those payloads to nearest with each 32-column run carrying its error (`encode_e4m3`,
    `:163-197`), the same bytes on every bake."""
    if grid not in GRIDS:
        raise ValueError(f"no grid {grid!r}")
    feedback = rounding == "feedback"
    flags = 0 if feedback else _rounding_flags(rounding)
    seed = _noise_seed(torch, seed, generator, rounding == "stochastic")
    up_a = _scaled_up(torch, up, alpha)
    raw, scales = data.view(torch.uint8), scale.view(-1)
    if scales.dtype != torch.float32 or not scales.is_contiguous():
        raise ValueError("a row-scaled bake keeps a contiguous float32 row scale")
    up32, down32 = up_a.to(torch.float32).contiguous(), down.to(torch.float32).contiguous()
    more_rows = _more_rows(torch, more, raw.shape[0], False)
    ops = _ops(raw)
    began = time.perf_counter()
    before = None if stats is None else {"data": raw.clone(), "scale": scales.clone()}
    if grid == "keep":
        new = scales.clone()
    else:
        amax = ops.bake_norms(ROWWISE, raw, scales, up32, down32, cols=raw.shape[1], amax=True, more=more_rows)
        # amax / 448 as torch runs it on a GPU (the reference's eager bake included): times the
        # float32 reciprocal, written out so that it does not depend on that detail.
        new = (amax * (1.0 / E4M3_MAX)).clamp(min=ROW_SCALE_FLOOR)
    if grid == "regrid":
        row = torch.arange(raw.shape[0], device=raw.device, dtype=torch.float32)
        new = new * (1 + (1 + 2 * torch.frac(row * 0.6180339887)) / 32)
    new = new.contiguous()
    if feedback:
        # Each element's nearest-rounding error carried into the next of its 32-column run, the
        # eager law's order `(decode · scale + delta) / new` on every grid, `keep`'s included.
        ops.bake_feedback(raw, scales, up32, down32, new, more=more_rows)
    else:
        # `keep` too bakes onto a row scale (the kept one), for the eager order above.
        ops.bake(ROWWISE, raw, scales, up32, down32, seed & SEED_MASK, more=more_rows, flags=flags, rescale=new)
    scales.copy_(new)
    if stats is not None:
        _account(torch, stats, ROWWISE, before, {"data": raw, "scale": scales}, up32, down32, raw.shape[1],
                 None, more_rows, began)  # fmt: skip


def bake_int8_convrot(torch: Any, data: Tensor, scale: Tensor, down: Tensor, up: Tensor, alpha: float, *,
                      rounding: str = "nearest", generator: Any = None, stats: Any = None,
                      more: Dense | None = None, seed: int | None = None) -> None:  # fmt: skip
    """Bake into `int8-convrot256/1` (`internal/lora_bake.py:372-423`): `down` and the dense
    rows rotated into the weight's basis, the row scale kept, nearest or stochastic floor,
    clamped to ±127."""
    flags = _rounding_flags(rounding)
    seed = _noise_seed(torch, seed, generator, flags == 0)
    fused(torch, {"weight": data, "scale": scale}, down, _scaled_up(torch, up, alpha), seed, more=more,
          flags=flags, stats=stats)  # fmt: skip


def bake_nvfp4(torch: Any, weight: Tensor, scale: Tensor, scale_2: Tensor, down: Tensor, up: Tensor,
               alpha: float, *, rounding: str = "stochastic", grid: str = "keep", generator: Any = None,
               stats: Any = None, more: Dense | None = None, gain: Tensor | None = None,
               seed: int | None = None) -> None:  # fmt: skip
    """Bake into canonical `nvfp4` (`internal/lora_bake.py:458-525`). `keep`: the second level
    kept and a block's scale refitted only past 7/6 of it. `refit`: the second level set from
    the baked tensor's amax and every block's scale from its own, saturation-free; `regrid` is
    `refit` (the reference branches on `grid != "keep"`, `:498`)."""
    if grid not in GRIDS:
        raise ValueError(f"no grid {grid!r}")
    flags = _rounding_flags(rounding)
    seed = _noise_seed(torch, seed, generator, flags == 0)
    if grid != "keep":
        _bake_nvfp4_refit(torch, weight, scale, scale_2, down, up, alpha, flags=flags, seed=seed, stats=stats,
                          more=more, gain=gain)  # fmt: skip
        return
    extra = gain is not None or more is not None or flags
    stored = {"weight": weight, "scale": scale, "scale_2": scale_2}
    if extra or rounding != "stochastic":
        fused(torch, stored, down, _scaled_up(torch, up, alpha), seed, gain=gain, more=more, flags=flags,
              stats=stats)  # fmt: skip
    else:
        # Without additions the eager law's separate roundings still apply (`base + delta`).
        ones = torch.ones(weight.shape[0], dtype=torch.float32, device=weight.device)
        fused(torch, stored, down, _scaled_up(torch, up, alpha), seed, gain=ones, stats=stats)


def _bake_nvfp4_refit(torch: Any, weight: Tensor, scale: Tensor, scale_2: Tensor, down: Tensor, up: Tensor,
                      alpha: float, *, flags: int, seed: int, stats: Any, more: Dense | None,
                      gain: Tensor | None) -> None:  # fmt: skip
    """`bake_nvfp4(grid="refit")` (`internal/lora_bake.py:495-525`): the baked tensor's amax (the
    row maxima of `cozyq_bake_row_amax` over `gain · decode + up @ down + more`, then their
    maximum) sets the new second level `amax / 2688` in float64 (1 for all zeros), and one launch
    refits every block on it. `Stats` decode the weight before at the stored level and after at
    the new one."""
    began = time.perf_counter()
    raw, blocks = weight.view(torch.uint8), scale.view(torch.uint8)
    rows, cols = int(raw.shape[0]), 2 * int(raw.shape[1])
    up32 = _scaled_up(torch, up, alpha).to(torch.float32).contiguous()
    down32 = down.to(torch.float32).contiguous()
    gain32 = None if gain is None else gain.to(torch.float32).reshape(-1).contiguous()
    more_rows = _more_rows(torch, more, rows, False)
    # A copy: `second` must keep the stored level while `scale_2` takes the new one.
    second = scale_2.to(torch.float32).reshape(-1)[:1].clone()
    ops = _ops(raw)
    stored_second = float(second[0])
    before = None if stats is None else {"data": raw.clone(), "blocks": blocks.clone(), "second": second}
    amax = 0.0
    if rows and cols:
        amax = float(ops.bake_norms(NVFP4, raw, None, up32, down32, cols=cols, blocks=blocks, second=second,
                                    amax=True, gain=gain32, more=more_rows).max())  # fmt: skip
    level = amax / (E4M3_MAX * 6.0) if amax > 0 else 1.0
    ops.bake_nvfp4_refit(raw, blocks, second, up32, down32, seed & SEED_MASK, level, flags=flags, gain=gain32,
                         more=more_rows)  # fmt: skip
    if level != stored_second:
        scale_2.copy_(torch.full_like(scale_2, level))
    if stats is not None:
        after = {"data": raw, "blocks": blocks,
                 "second": torch.full((1,), level, dtype=torch.float32, device=raw.device)}  # fmt: skip
        _account(torch, stats, NVFP4, before, after, up32, down32, cols, gain32, more_rows, began)


def warm(torch: Any, device: int) -> None:
    """The bake kernels are part of `libcozyq.so` and serve from the first call
    (`internal/lora_bake.py:817-821` builds Triton kernels here): opening the library is all."""
    serving(torch, device)


def serving(torch: Any, device: int) -> str:
    """How a bake on GPU `device` runs (`internal/lora_bake.py:824-835`): always `fused`, the
    HIP kernels; the library opens (or raises) here."""
    from cozyq import prebuilt

    prebuilt.library(device)
    return "fused"


def rotate_rows(torch: Any, rows: Dense) -> Dense:
    """`rows` in an `int8-convrot256/1` weight's basis, as `rotate_factor` rotates `down`
    (`internal/lora_bake.py:648-650`)."""
    return lambda start, stop: rotate_factor(torch, rows(start, stop))


def norms(torch: Any, stored: Mapping[str, Tensor], down: Tensor, up: Tensor) -> Tensor:
    """Each output row's L2 norm of a linear's stored weight plus `up @ down`, float32 `[out]`
    (`internal/lora_bake.py:653-689`). An `int8-convrot256/1` weight's rows are rotated, and so is
    the delta: the rotation is orthonormal, so the norm is the unrotated weight's."""
    up32 = up.to(torch.float32).contiguous()
    down32 = down.to(torch.float32).contiguous()
    if "scale_2" in stored:
        raw = stored["weight"].view(torch.uint8)
        second = stored["scale_2"].to(torch.float32).reshape(1)
        return _ops(raw).bake_norms(NVFP4, raw, None, up32, down32, cols=2 * raw.shape[1],
                                    blocks=stored["scale"].view(torch.uint8), second=second)  # fmt: skip
    if "value" in stored:
        value = stored["value"]
        kind = {torch.bfloat16: BF16, torch.float16: F16, torch.float32: F32}[value.dtype]
        return _ops(value).bake_norms(kind, value, None, up32, down32, cols=value.shape[1])
    data, scale = stored["weight"], stored["scale"].reshape(-1).to(torch.float32).contiguous()
    if data.dtype == torch.int8:
        return _ops(data).bake_norms(INT8, data, scale, up32, rotate_factor(torch, down32),
                                     cols=data.shape[1])  # fmt: skip
    raw = data.view(torch.uint8)
    return _ops(raw).bake_norms(ROWWISE, raw, scale, up32, down32, cols=raw.shape[1])


def dora_ratio(torch: Any, magnitude: Tensor, norm: Tensor) -> Tensor:
    """`m / ||V||` per output row, float32; 0 where `V`'s row is 0
    (`internal/lora_bake.py:692-695`)."""
    tiny = torch.finfo(torch.float32).tiny
    return torch.where(norm > 0, magnitude.float() / norm.clamp_min(tiny), 0.0)


def dora_weight(torch: Any, weight: Tensor, down: Tensor, up: Tensor, magnitude: Tensor,
                s: float, t: float) -> Tensor:  # fmt: skip
    """PEFT's DoRA weight at strength `t`, float32 `[out, in]`: `W + t * (m * V / ||V|| - W)`
    per output row, `V = W + s * B @ A` (`internal/lora_bake.py:698-712`)."""
    v = weight + (up.float() @ down.float()) * s
    ratio = dora_ratio(torch, magnitude, torch.linalg.vector_norm(v, dim=1))
    return weight + (v * ratio[:, None] - weight) * t


def dora(torch: Any, stored: Mapping[str, Tensor],
         terms: list[tuple[Tensor, Tensor, Tensor, float, float]]) -> tuple[Tensor, list[Tensor]]:  # fmt: skip
    """A stored linear's DoRA terms, each `(A, B, m, s, t)`, as its row gain and each term's B
    scale (float32 `[out]`, `internal/lora_bake.py:715-730`): `g = 1 + t * (r - 1)` and
    `c = t * s * r` with `r = m / ||V||`, the norms taken from the stored rows (`norms`)."""
    gain = torch.ones_like(terms[0][2], dtype=torch.float32)
    scales = []
    for down, up, magnitude, s, t in terms:
        ratio = dora_ratio(torch, magnitude, norms(torch, stored, down, up.float() * s))
        gain.add_(ratio - 1, alpha=t)
        scales.append(ratio.mul_(t * s))
    return gain, scales


def gain_rows(torch: Any, stored: dict[str, Tensor], gain: Tensor) -> None:
    """Each output row of a stored weight times `gain` (float32 `[out]`), in place
    (`internal/lora_bake.py:733-749`): a row-scaled weight's scale exactly, a plain one's values
    rounded once to nearest, an nvfp4 one's re-encoded (`bake_nvfp4` with no delta, nearest)."""
    gain32 = gain.to(torch.float32).reshape(-1).contiguous()
    if "scale_2" not in stored and "value" not in stored:
        stored["scale"].view(-1).mul_(gain32)
        return
    probe = stored["weight"] if "scale_2" in stored else stored["value"]
    cols = 2 * probe.shape[1] if "scale_2" in stored else probe.shape[1]
    down = torch.zeros((0, cols), dtype=torch.float32, device=probe.device)
    up = torch.zeros((probe.shape[0], 0), dtype=torch.float32, device=probe.device)
    fused(torch, stored, down, up, 0, gain=gain32, flags=NEAREST | NO_DELTA)


def accumulate(torch: Any, x: Tensor, out: Tensor, down: Tensor, up: Tensor, alpha: float) -> None:
    """`out += alpha * (x @ down.T) @ up.T` in two library GEMMs (`internal/lora_bake.py:
    752-761`): the up projection adds into the base output, so no `[rows, out]` update is ever
    allocated."""
    flat, rows = out.view(-1, out.shape[-1]), x.reshape(-1, x.shape[-1])
    low = torch.nn.functional.linear(rows, down.to(rows.dtype))
    flat.addmm_(low.to(flat.dtype), up.to(flat.dtype).t(), alpha=alpha)


def recipe(fused: bool = True) -> str:
    """What names the bytes a bake writes to other executors (`internal/lora_bake.py:846-850`):
    `VARIANT` and the path it bakes by."""
    if not fused:
        raise NotImplementedError("cozyq has no eager bake")
    return f"{VARIANT} fused gfx950 philox4x32-10"


def probe(torch: Any, device: Any) -> Verdict:
    """Bake every form on `device` where the result is exact (`internal/lora_bake.py:852-898`:
    0.25 + 24·(±1/32) is 1.0 or −0.5, over partial tiles and two inner steps): one stored value
    off it is a broken kernel."""
    rows, cols, rank = 70, 96, 24
    f32 = torch.float32
    up = torch.full((rows, rank), 1 / 32, device=device, dtype=f32)
    up[1::2] = -1 / 32
    down = torch.ones((rank, cols), device=device, dtype=f32)
    halves = torch.tensor([1.0, -0.5], device=device, dtype=f32).repeat(rows // 2)[:, None]
    want = halves.expand(rows, cols)
    wrong: dict[int, int] = {}
    for kind in (BF16, F16, F32, ROWWISE):
        if kind == ROWWISE:
            data = torch.full((rows, cols), 0.5, device=device, dtype=f32).to(torch.float8_e4m3fn)
            stored = {"weight": data, "scale": torch.full((rows,), 0.5, device=device, dtype=f32)}
        else:
            dtype = (torch.bfloat16, torch.float16, torch.float32)[kind]
            stored = {"value": torch.full((rows, cols), 0.25, dtype=dtype, device=device)}
        fused(torch, stored, down, up, kind)
        got = stored["value"].float() if "value" in stored else stored["weight"].float() * 0.5
        wrong[kind] = int((got != want).sum())
    nv = {
        "weight": torch.full((rows, cols // 2), 0x11, dtype=torch.uint8, device=device),
        "scale": torch.full((rows, cols // 16), 0.5, device=device, dtype=f32).to(torch.float8_e4m3fn),
        "scale_2": torch.ones(1, device=device, dtype=f32),
    }
    fused(torch, nv, down, up, NVFP4)
    grid = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], device=device, dtype=f32)
    grid = torch.cat((grid, -grid))
    raw = nv["weight"]
    codes = torch.stack((raw & 15, raw >> 4), dim=-1).reshape(rows, cols).long()
    got = grid[codes] * nv["scale"].float().repeat_interleave(16, dim=1)
    wrong[NVFP4] = int((got != want).sum())
    data = torch.full((rows, 256), 2, dtype=torch.int8, device=device)
    stored = {"weight": data, "scale": torch.full((rows,), 0.5, device=device, dtype=f32)}
    fused(torch, stored, torch.ones((rank, 256), device=device, dtype=f32), up * (32 / 48), INT8)
    ints = torch.tensor([3, 1], device=device).repeat(rows // 2)[:, None].expand(rows, 256)
    wrong[INT8] = int((data.long() != ints).sum())
    off = {kind: n for kind, n in wrong.items() if n}
    detail = f"form(s) {off} stored values off the grid" if off else f"{len(wrong)} forms exact"
    return Verdict(not off, detail)

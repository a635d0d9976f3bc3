"""The LoRA bake on gfx950: cozyq's counterpart of cozy-runtime's `internal/lora_bake.py`.

A LoRA's `up @ down` is added into a stored weight in place and rounded back onto the weight's
own form, so that the adapted layer serves at the speed of the unadapted one. The reference
bakes on the GPU with one Triton kernel per stored form (`fused`, `:775-815`); this module keeps
its surface — `bakeable`, `rotate_factor`, `fused`, `bake`, `probe`, `recipe` and the form
constants — with the kernels in `csrc/bake.hip` behind `cozyq_bake`, `cozyq_bake_nvfp4` and
`cozyq_bake_rotate_factor`:

* plain bf16 (stochastic: 16 noise bits added under the kept ones), f16 and f32 (nearest);
* `fp8.rowwise` (E4M3 data, stochastic, row scale kept);
* `int8-convrot256/1` (int8 of the rotated rows, stochastic floor, row scale kept; `down` is
  rotated into the weight's basis first);
* canonical `nvfp4` (E2M1 codes on the kept block grid, a block's E4M3 scale refitted only when
  its baked maximum outgrows 7/6 of it, the second level kept).

Element (row, col)'s noise is Triton's Philox draw at counter `row * cols + col` under the
weight's 31-bit seed, and the delta is one float32 FMA chain in rank order, so a bake writes the
bytes the reference's fused bake writes for the same factors.

Not built: the reference's eager bake (`bake_plain`, `bake_rowwise`, `bake_int8_convrot`,
`bake_nvfp4` over torch's generator), which serves `Stats`, `refit` / `regrid` grids, nearest and
feedback rounding, a DoRA gain on plain or nvfp4 rows and LoKr rows (`more`); asking for any of
them raises NotImplementedError. A DoRA gain on a row-scaled weight folds into its scale, as the
reference does. Tensors off the GPU raise.
"""

from __future__ import annotations

from collections.abc import Mapping
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


class Verdict(NamedTuple):
    ok: bool
    detail: str


def bakeable(scheme: str, params: Mapping[str, object], roles: Mapping[str, str]) -> bool:
    """Whether a stored weight (scheme, params, role → dtype) takes `bake`
    (`internal/lora_bake.py:537-551`): plain bf16 / f16 / f32, `fp8.rowwise` E4M3 with a float32
    row scale, canonical `nvfp4` (its activation `input_scale` aside) or `int8.convrot`. An
    int8.convrot weight must carry the 256 rotation the bake rotates `down` by; the reference
    does not ask and would bake a smaller rotation's weight in the wrong basis."""
    if scheme == "plain":
        return dict(roles) in ({"value": "bf16"}, {"value": "f16"}, {"value": "f32"})
    if scheme == "fp8.rowwise":
        return dict(roles) == {"weight": "f8_e4m3fn", "scale": "f32"}
    if scheme == "nvfp4":
        kept = {role: dtype for role, dtype in roles.items() if role != "input_scale"}
        return kept == {"weight": "u8", "scale": "f8_e4m3fn", "scale_2": "f32"} and all(
            params.get(name, value) == value for name, value in NVFP4_PARAMS.items()
        )
    return (
        scheme == "int8.convrot"
        and dict(roles) == {"weight": "i8", "scale": "f32"}
        and int(dict(params).get("rotation_size", CONVROT_GROUP)) == CONVROT_GROUP  # type: ignore[call-overload]
    )


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


def fused(torch: Any, stored: dict[str, Tensor], down: Tensor, up: Tensor, seed: int) -> None:
    """`bake`, one kernel launch (`internal/lora_bake.py:775-815`): each tile adds its
    `up @ down` (float32) to the decoded stored values and rounds them back in place."""
    up32 = up.to(torch.float32).contiguous()
    down32 = down.to(torch.float32).contiguous()
    if "scale_2" in stored:
        raw = stored["weight"].view(torch.uint8)
        second = stored["scale_2"].to(torch.float32).reshape(1)
        _ops(raw).bake_nvfp4(raw, stored["scale"].view(torch.uint8), second, up32, down32,
                             seed & SEED_MASK)  # fmt: skip
        return
    if "value" in stored:
        data = stored["value"]
        kinds = {torch.bfloat16: BF16, torch.float16: F16, torch.float32: F32}
        if data.dtype not in kinds:
            raise ValueError(f"a plain bake stores bf16, f16 or f32, not {data.dtype}")
        kind, scale = kinds[data.dtype], None
    elif stored["weight"].dtype == torch.int8:
        data, scale, kind = stored["weight"], stored["scale"].reshape(-1), INT8
        down32 = rotate_factor(torch, down32)
    else:
        data, scale, kind = stored["weight"].view(torch.uint8), stored["scale"].reshape(-1), ROWWISE
    if scale is not None and (scale.dtype != torch.float32 or not scale.is_contiguous()):
        raise ValueError("a row-scaled bake keeps a contiguous float32 row scale")
    _ops(data).bake(kind, data, scale, up32, down32, seed & SEED_MASK)


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
    more: Any = None,
) -> None:
    """Bake `up @ down` into one stored weight by its roles (`internal/lora_bake.py:554-645`):
    plain floats, `fp8.rowwise`, `int8-convrot256/1` or canonical `nvfp4`. A convolution's weight
    and factors bake as matrices, each kernel tap one more input column. `gain` (float32 per
    output row, a DoRA's) on a row-scaled weight multiplies its scale exactly; `seed` names the
    weight's noise. `down` and `up` may have rank 0."""
    if down.dim() > 2:
        stored = {role: t.view(t.shape[0], -1) if t.dim() > 2 else t for role, t in stored.items()}
        down, up = down.flatten(1), up.flatten(1)
    if gain is not None and "value" not in stored and "scale_2" not in stored:
        stored["scale"].view(-1).mul_(gain)
        gain = None
    if stats is not None or gain is not None or more is not None or how not in ("fused", None):
        raise NotImplementedError(
            "cozyq bakes by the fused law only: Stats, a DoRA gain on plain or nvfp4 rows, LoKr "
            "rows and the eager reference bake are not built"
        )
    fused(torch, stored, down, up, seed)


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

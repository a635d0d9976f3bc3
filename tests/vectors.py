"""Reading the reference's decode vectors (`tests/golden/ref_*_vectors.json`): parts as torch
tensors in the runtime's form (an `F4` part as its packed bytes `[..., C/2]`, E8M0 as uint8),
the expected output bytes, and bit-for-bit comparison (any NaN matches any NaN)."""

from __future__ import annotations

import base64
import json
from pathlib import Path

import torch

GOLDEN = Path(__file__).resolve().parent / "golden"
DTYPES = {"F32": torch.float32, "BF16": torch.bfloat16, "F16": torch.float16, "I8": torch.int8,
          "F8_E4M3": torch.float8_e4m3fn, "F8_E5M2": torch.float8_e5m2, "F8_E8M0": torch.uint8,
          "F4": torch.uint8, "U8": torch.uint8}  # fmt: skip
#: JSON dtype names → the runtime names `cozyq.decode.part_rule` reads; others pass through.
NAMES = {"F32": "f32", "BF16": "bf16", "F16": "f16", "I8": "i8", "F8_E4M3": "f8_e4m3fn",
         "F8_E5M2": "f8_e5m2", "F8_E8M0": "f8_e8m0", "F4": "u8", "U8": "u8", "I32": "i32"}  # fmt: skip


def stored_shape(dtype: str, shape: list[int]) -> list[int]:
    return [*shape[:-1], shape[-1] // 2] if dtype == "F4" and shape else list(shape)


def tensor(bits: str, dtype: str, shape: list[int]) -> torch.Tensor:
    raw = bytearray(base64.b64decode(bits))
    shape = stored_shape(dtype, shape)
    if not raw:
        return torch.empty(shape, dtype=DTYPES[dtype])
    return torch.frombuffer(raw, dtype=DTYPES[dtype]).reshape(shape)


def cases(name: str, component: str | None = None) -> list[dict]:
    data = json.loads((GOLDEN / f"ref_{name}_vectors.json").read_text())
    return [c for c in data["cases"] if component is None or c["component"] == component]


def parts(case: dict) -> dict[str, torch.Tensor]:
    return {p["role"]: tensor(p["bits"], p["dtype"], p["shape"]) for p in case["parts"]}


def part_names(case: dict) -> dict[str, tuple[str, list[int]]]:
    """Each part's runtime dtype name and stored shape, as the fill plane sees them."""
    return {p["role"]: (NAMES.get(p["dtype"], p["dtype"]), stored_shape(p["dtype"], p["shape"]))
            for p in case["parts"]}  # fmt: skip


def expected(case: dict, dtype: torch.dtype) -> torch.Tensor:
    return torch.frombuffer(bytearray(base64.b64decode(case["expect"])), dtype=dtype).reshape(
        case["shape"])


def same(got: torch.Tensor, case: dict) -> bool:
    """Bit-for-bit equality with the case's expected output; a NaN matches any NaN (NaN payloads
    are not part of any decode law)."""
    got = got.cpu()
    want = expected(case, got.dtype)
    nan = torch.isnan(got.float())
    if not torch.equal(nan, torch.isnan(want.float())):
        return False
    bits = torch.int32 if got.element_size() == 4 else torch.int16
    return torch.equal(got[~nan].contiguous().view(bits), want[~nan].contiguous().view(bits))

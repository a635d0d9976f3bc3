"""The card's self-check: before the op library serves on a card, each format's kernels run on
it against that format's exact law in float64, and a failing format refuses the library (there
is no other lane to fall back to, so it raises). cozyq's counterpart of cozy-runtime's
`internal/verify.py` (relative L2 against the law, `:70-104`; crash markers, `:110-175`) and the
probe of `internal/prebuilt.py:601-675`.

- `probe_int8` / `probe_fp8` run the serving entry points on small problems: the linear at a
  GEMV-sized and a GEMM-sized M, the GEMM's shape rule at the GEMV-sized M, bf16 and fp16, and
  every GEMM tile config on the same operand (int8's integer sums must give every config the
  same bits).
- Their law is restated here in float64 on the device (the format definitions: per-token int8
  of the 256-point rotated rows, `internal/int8_linear.py:422-428`, and per-token e4m3,
  `internal/fp8_linear.py:56-63`). A kernel that rounds the same law its own way loses ~2^-9 to
  its output dtype; garbage loses O(1). `BUDGET` sits between.
- A probe that ends its process (a device fault) leaves its marker behind; the next process on
  the machine finds it and refuses that format without running it again. Delete the marker
  (the refusal names it) to probe again.
"""

from __future__ import annotations

import fcntl
import hashlib
import math
import os
from collections.abc import Callable
from dataclasses import dataclass
from pathlib import Path
from typing import Any

Tensor = Any

#: Relative L2 error a served kernel may show against its format's law.
BUDGET = 1e-2
#: What a refusal for a probe that ended an earlier process says.
CRASHED = "its self-check ended an earlier process on this machine"


@dataclass(frozen=True)
class Verdict:
    """A format's self-check: whether it serves, and what was measured or why it failed."""

    ok: bool
    detail: str


def error(torch: Any, got: Tensor, want: Tensor) -> float:
    """Relative L2 error of `got` against `want` in float64; inf where `got` is not finite."""
    got = got.double()
    if not bool(torch.isfinite(got).all()):
        return math.inf
    want = want.double()
    return float((got - want).norm() / want.norm().clamp(min=1e-30))


def within(errors: dict[str, float], budget: float = BUDGET) -> Verdict:
    """Every case within `budget`, said with the worst one; no cases is a failure."""
    if not errors:
        return Verdict(False, "no case ran")
    worst = max(errors, key=lambda case: errors[case])
    detail = f"rel L2 {errors[worst]:.2e} at {worst} (budget {budget:g}, {len(errors)} cases)"
    return Verdict(errors[worst] <= budget, detail)


# ------------------------------------------------------------------ verdicts and markers

#: key -> verdict, for this process.
_KNOWN: dict[str, Verdict] = {}


def marker_dir() -> Path | None:
    """Where probe markers live: `$COZYQ_VERIFY_DIR`, else `~/.cache/cozyq/verify`; None where
    neither can be made (the probe then runs unguarded)."""
    root = os.environ.get("COZYQ_VERIFY_DIR")
    path = Path(root) if root else Path.home() / ".cache" / "cozyq" / "verify"
    try:
        path.mkdir(parents=True, exist_ok=True)
    except OSError:
        return None
    return path


def library_digest(path: Path) -> str:
    """The first 16 hex digits of the library file's SHA-256: a rebuilt library probes anew."""
    digest = hashlib.sha256()
    with path.open("rb") as fh:
        for block in iter(lambda: fh.read(1 << 20), b""):
            digest.update(block)
    return digest.hexdigest()[:16]


def verified(key: str, probe: Callable[[], Verdict], device_fault: Callable[[], str] = lambda: "") -> Verdict:
    """`key`'s verdict for this process: probed now (once), unless a probe of it ended an earlier
    process on this machine. A probe that raises fails with its exception; `device_fault` says,
    after the probe, whether the device context died under it (then the marker is kept)."""
    known = _KNOWN.get(key)
    if known is None:
        known = _KNOWN[key] = _probed(key, probe, device_fault)
    return known


def _run(probe: Callable[[], Verdict]) -> Verdict:
    try:
        return probe()
    except Exception as exc:  # a probe that raises fails, with why
        return Verdict(False, f"the probe raised {type(exc).__name__}: {exc}"[:400])


def _probed(key: str, probe: Callable[[], Verdict], device_fault: Callable[[], str]) -> Verdict:
    folder = marker_dir()
    if folder is None:
        return _run(probe)
    marker = folder / f"{key}.probing"
    try:
        lock = (folder / f"{key}.lock").open("a+")
    except OSError:
        return _run(probe)
    with lock:
        # Another process of this machine probing the same key finishes first; a lock dies with
        # its process, so a marker found while holding it was left by a probe that never ended.
        fcntl.flock(lock, fcntl.LOCK_EX)
        if marker.exists():
            return Verdict(False, f"{CRASHED} (marker {marker}: {marker.read_text()[:200]})")
        marker.write_text(f"pid {os.getpid()} probing\n")
        fault = ""
        try:
            verdict = _run(probe)
            fault = device_fault()
            if fault:
                verdict = Verdict(False, f"the device faulted under the probe: {fault}"[:400])
            return verdict
        finally:
            if fault:
                marker.write_text(f"pid {os.getpid()}: the device faulted under the probe: {fault}\n")
            else:
                marker.unlink(missing_ok=True)


def cuda_fault(torch: Any) -> Callable[[], str]:
    """Why the device context is dead after a probe, else empty (a wild launch kills the context,
    and the next synchronization raises)."""

    def check() -> str:
        try:
            torch.cuda.synchronize()
        except Exception as exc:  # the context is gone
            return f"{type(exc).__name__}: {exc}"
        return ""

    return check


# ------------------------------------------------------------------ the formats' laws

#: The 4-point stage of the reference's rotation (outer digit first, rows are outputs):
#: (a, b, c, d) -> (a+b+c-d, a+b-c+d, a-b+c+d, b+c+d-a) (`internal/encoding/formats.py:657-671`).
_STAGE = ((1, 1, 1, -1), (1, 1, -1, 1), (1, -1, 1, 1), (-1, 1, 1, 1))


def rotation(torch: Any, device: Any) -> Tensor:
    """The 256-point rotation as a float64 matrix, 1/16 applied (orthonormal): four 4-point
    stages, one per base-4 digit of the index. The stage matrix is symmetric, and so is this."""
    stage = torch.tensor(_STAGE, dtype=torch.float64, device=device)
    full = stage
    for _ in range(3):
        full = torch.kron(full, stage)
    return full / 16.0


def int8_law(torch: Any, x: Tensor, data: Tensor, scale: Tensor, bias: Tensor | None) -> Tensor:
    """int8.convrot's product in float64: each 256-group of a row rotated, s = max(amax / 127,
    1e-12), q = clamp(rne(r / s), ±127); out = (q · dataᵀ) · s · scale + bias."""
    rows, width = x.shape
    r = (x.double().reshape(rows, width // 256, 256) @ rotation(torch, x.device)).reshape(rows, width)
    s = (r.abs().amax(-1, keepdim=True) / 127.0).clamp(min=1e-12)
    q = torch.round(r / s).clamp(-127, 127)
    out = (q @ data.double().t()) * s * scale.double().reshape(1, -1)
    return out if bias is None else out + bias.double()


def fp8_law(torch: Any, x: Tensor, data: Tensor, scale: Tensor, bias: Tensor | None) -> Tensor:
    """fp8.rowwise's product in float64: s = max(amax / 448, 1e-12) in float32, q =
    e4m3(clamp(x / s, ±448)); out = (q · dataᵀ) · s · scale + bias."""
    s = (x.abs().amax(-1, keepdim=True).float() / 448.0).clamp(min=1e-12)
    q = (x.float() / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    out = (q.double() @ data.double().t()) * s.double() * scale.double().reshape(1, -1)
    return out if bias is None else out + bias.double()


# ------------------------------------------------------------------ the probes

#: The probes' shape: rows for the GEMM path, output features, width (every lane's K).
ROWS, FEATURES, WIDTH = 300, 512, 1024


def _probe(torch: Any, ops: Any, fp8: bool) -> Verdict:
    device = torch.device("cuda", ops.index)
    gen = torch.Generator(device=device).manual_seed(20261202)

    def randn(*shape: int, scale: float = 1.0) -> Tensor:
        return torch.randn(*shape, generator=gen, device=device, dtype=torch.float32) * scale

    if fp8:
        data = randn(FEATURES, WIDTH, scale=60.0).clamp(-448, 448).to(torch.float8_e4m3fn)
        linear, gemm, quantize, law = ops.fp8_linear, ops.fp8_gemm, ops.fp8_quantize, fp8_law
        few = (3, 12)  # the GEMV and the row-tile kernel
    else:
        data = torch.randint(-127, 128, (FEATURES, WIDTH), generator=gen, device=device, dtype=torch.int8)
        linear, gemm, quantize, law = ops.int8_linear, ops.int8_gemm, ops.int8_quantize, int8_law
        few = (3,)
    scale = randn(FEATURES).abs().add(0.5).mul(1e-3)
    errors: dict[str, float] = {}
    from cozyq.prebuilt import GEMM_CONFIGS as configs
    for dtype in (torch.bfloat16, torch.float16):
        name = "bf16" if dtype == torch.bfloat16 else "fp16"
        bias = randn(FEATURES).to(dtype)
        x = want = None
        for m in (*few, ROWS):
            x = randn(m, WIDTH).to(dtype)
            want = law(torch, x, data, scale, bias)
            errors[f"{name} linear M={m}"] = error(torch, linear(x, data, scale, bias, dtype), want)
            if m < ROWS:  # the shape rule's GEMM on few quantized rows
                qm, sm = quantize(x)
                errors[f"{name} GEMM M={m}"] = error(torch, gemm(qm, sm, data, scale, bias, dtype, -1), want)
        q, s = quantize(x)
        first = None
        for config in range(configs):
            got = gemm(q, s, data, scale, bias, dtype, config)
            errors[f"{name} tile {config}"] = error(torch, got, want)
            if first is None:
                first = got
            elif not torch.equal(got, first):
                errors[f"{name} tile {config} bits differ from tile 0"] = math.inf
    return within(errors)


def probe_int8(torch: Any, ops: Any) -> Verdict:
    """int8.convrot's kernels on the card: the linear at M = 3 (the fused GEMV) and 300
    (quantize + the shape rule's GEMM), the GEMM at M = 3 (the GEMV on the quantized rows), bf16
    and fp16, and every tile config bit-equal."""
    return _probe(torch, ops, fp8=False)


def probe_fp8(torch: Any, ops: Any) -> Verdict:
    """fp8.rowwise's kernels on the card: the linear at M = 3 (GEMV), 12 (the row-tile kernel)
    and 300 (quantize + GEMM), bf16 and fp16, and every tile config (each within budget; the
    configs share one MFMA order, so they agree too)."""
    return _probe(torch, ops, fp8=True)


#: The formats the library verifies before it serves, and their probes.
PROBES: dict[str, Callable[[Any, Any], Verdict]] = {"int8": probe_int8, "fp8": probe_fp8}

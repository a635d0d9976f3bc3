"""Benchmark of the quantized-linear hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra]

Headline: one step = the block-Hadamard rotation (128) + per-token int8
quantization of X [4096, 3072] and the W8A8 int8 GEMM against W [12288, 3072] with the bias and
tanh-GELU epilogue, bf16 out. `value` is TOPS over the whole step (2·M·N·K ops), inputs resident
in HBM. `roofline` is the GEMM kernel's achieved int8 TOPS (timed alone with HIP events on the
launch stream) against the 5.0 POPS dense int8 MFMA peak. `decode` is BASELINE's second target:
the fp8 rowwise linear at M=1, K=4096, N=14336 (quantize + GEMV fused in one launch), in HBM GB/s
against 8 TB/s, rotating 8 weight copies (470 MB) so the 256 MB MALL cannot hold them.
`configs` reports the other BASELINE configs. `cpu_baseline` times the reference's CPU law
(the oracle's restatement of internal/int8_linear.py:415-448, its literal int32 matmul) on a
bounded sample of the same workload on this host's cores; `cpu_baselines` does so for every
config.

Timing: a fixed clock pre-roll (PREROLL_MS of the C2 step, whatever --warmup says), then the
driver's contract for `value` (W warm-up steps, K steps between two synchronizations); every
other figure is the median of SAMPLES interleaved samples (HIP events on the launch stream).

Prints one JSON line. Only one GPU is used; `--gpus` above 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "cozy-runtime_amd"))

METRIC = "quantized-linear TOPS & % MFMA peak (M=4096,K=3072,N=12288); M=1 HBM GB/s"
#: MI355X datasheet peaks (dense): int8 5.0 POPS, fp8 5.0 PFLOPS, bf16 2.5 PFLOPS, HBM 8 TB/s.
PEAK_INT8_TOPS = 5000.0
PEAK_FP8_TFLOPS = 5000.0
PEAK_BF16_TFLOPS = 2500.0  # dense bf16 / fp16 MFMA
PEAK_HBM_GBS = 8000.0
#: HBM bytes per launch come from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs (one counter a
#: pass, each scaled by the same counter's reading for a 256 MiB device copy), whose summary
#: table is committed here; `roofline.traffic` is read from it by kernel name (null if absent).
PMC_SUMMARY = ROOT / "profiles" / "hbm_traffic_pmc.txt"
#: Timed samples per figure (medians are reported) and the clock pre-roll before any timing.
SAMPLES = 15
PREROLL_MS = 60.0


def pmc_traffic(leg: str, kernel: str) -> dict | None:
    """HBM bytes per dispatch of `kernel` (its demangled name's prefix) in leg `leg` of the
    committed PMC summary: {"read", "write", "total"} in bytes, or None."""
    try:
        lines = PMC_SUMMARY.read_text().splitlines()
    except OSError:
        return None
    for line in lines:
        cols = line.split()
        if len(cols) < 7 or cols[0] != leg:
            continue
        name = " ".join(cols[1:-5])
        if name.startswith(kernel):
            read, write = float(cols[-3]) * 1e6, float(cols[-1]) * 1e6
            return {"read": read, "write": write, "total": read + write,
                    "source": f"{PMC_SUMMARY.relative_to(ROOT)}: {name}"}
    return None


def _seeded(torch, seed: int):
    return torch.Generator(device="cuda").manual_seed(seed)


def _activations(torch, m: int, k: int, seed: int):
    """bf16 ~N(0,1) with 1% of the K channels scaled x20, generated on the device."""
    gen = _seeded(torch, seed)
    x = torch.randn(m, k, generator=gen, device="cuda")
    chans = torch.randperm(k, generator=gen, device="cuda")[: max(1, k // 100)]
    x[:, chans] *= 20
    return x.to(torch.bfloat16)


def _weights(torch, n: int, k: int, seed: int):
    return (torch.randn(n, k, generator=_seeded(torch, seed), device="cuda") * 0.02).to(torch.bfloat16)


class Timer:
    """HIP events on the launch stream (torch's current stream, which every launch here uses)."""

    def __init__(self, torch):
        self.torch = torch

    def run(self, fn, iters: int, warmup: int) -> float:
        """Average ms per call of `fn` over `iters` back-to-back calls after `warmup`."""
        torch = self.torch
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(iters):
            fn()
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / iters

    def interleaved(self, fns: dict, samples: int = SAMPLES, batch: int = 8) -> dict:
        """Per-call ms of each of `fns`: `samples` rounds, each timing `batch` back-to-back calls
        of every function in turn (candidates interleaved, as `internal/bench/gemm.py:370-392`
        does), so clock drift falls on all of them alike. Returns the median per function, with
        the fastest and slowest sample."""
        torch = self.torch
        events = {name: [] for name in fns}
        for _ in range(samples):
            for name, fn in fns.items():
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                for _ in range(batch):
                    fn()
                b.record()
                events[name].append((a, b))
        torch.cuda.synchronize()
        out = {}
        for name, pairs in events.items():
            ms = sorted(a.elapsed_time(b) / batch for a, b in pairs)
            out[name] = {"ms": ms[len(ms) // 2], "min_ms": ms[0], "max_ms": ms[-1], "samples": len(ms)}
        return out


def preroll(torch, fn, ms: float = PREROLL_MS) -> float:
    """Runs `fn` back to back for at least `ms` of wall time before anything is timed: the
    chip's clocks rise over the first ~20 ms of sustained MFMA load (the first 20-launch round
    of the C2 GEMM measured ~12% slower than later ones). Returns the wall ms spent."""
    start = time.perf_counter()
    while (time.perf_counter() - start) * 1e3 < ms:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()
    return (time.perf_counter() - start) * 1e3


def _check(code: int) -> None:
    if code != 0:
        from cozyq import _lib

        raise RuntimeError(f"kernel launch failed: {_lib.error_name(code)}")


def bench_c2(torch, ops, lib, stream, steps: int, warmup: int, preroll_for: float = PREROLL_MS) -> dict:
    m, k, n = 4096, 3072, 12288
    x = _activations(torch, m, k, 20261202)
    data, scale = ops.int8_quantize_rot(_weights(torch, n, k, 20261203), 128)
    bias = (torch.randn(n, generator=_seeded(torch, 5), device="cuda") * 0.1).to(torch.bfloat16)
    q = torch.empty(m, k, dtype=torch.int8, device="cuda")
    s = torch.empty(m, dtype=torch.float32, device="cuda")
    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    xp, qp, sp, dp, wp, bp, op = (t.data_ptr() for t in (x, q, s, data, scale, bias, out))

    def quantize():
        _check(lib.cozyq_quantize_rot(0, xp, 0, qp, sp, m, k, 128, stream))

    def gemm():
        _check(lib.cozyq_gemm_ex(0, 0, qp, sp, dp, wp, bp, op, n, 0, m, n, k, 1, stream))

    work = torch.zeros(int(lib.cozyq_linear_workspace_bytes(m)) // 4, dtype=torch.int32, device="cuda")

    def fused():
        # Rotation, quantization and the GEMM in one persistent launch (`cozyq_linear`).
        _check(lib.cozyq_linear(0, xp, 0, 128, qp, sp, dp, wp, bp, op, n, 0, m, n, k, 1,
                                work.data_ptr(), stream))  # fmt: skip

    def step():
        # The product path (`Prebuilt.int8_linear`): quantize, then the GEMM; faster than the
        # fused launch on MI355X.
        quantize()
        gemm()

    timer = Timer(torch)
    preroll_ms = preroll(torch, step, preroll_for)
    # The driver's contract: W untimed steps, then exactly K steps between two synchronizations.
    ms_step = timer.run(step, steps, warmup)

    # The same step at the reference's own rotation (256, regular H4^4, the parity-pinned one):
    # its weight rotated and quantized alike, the same GEMM and epilogue.
    data256, scale256 = ops.int8_quantize_rot(_weights(torch, n, k, 20261203), 256)
    dp256, wp256 = data256.data_ptr(), scale256.data_ptr()

    def step256():
        _check(lib.cozyq_quantize_rot(0, xp, 0, qp, sp, m, k, 256, stream))
        _check(lib.cozyq_gemm_ex(0, 0, qp, sp, dp256, wp256, bp, op, n, 0, m, n, k, 1, stream))

    med = timer.interleaved({"step": step, "gemm": gemm, "quantize": quantize, "fused": fused,
                             "step256": step256})
    ms_gemm, ms_quant, ms_step256 = med["gemm"]["ms"], med["quantize"]["ms"], med["step256"]["ms"]
    ops_count = 2.0 * m * n * k
    gemm_tops = ops_count / (ms_gemm * 1e-3) / 1e12
    traffic_alg = m * k + n * k + m * n * 2 + n * 2 + (m + n) * 4
    c2_traffic = pmc_traffic("c2", "void gemm8_kernel<0, false, true, 1>")
    return {
        "ms_per_step": ms_step,
        "tops": ops_count / (ms_step * 1e-3) / 1e12,
        "preroll_ms": preroll_ms,
        "step_median_ms": med["step"]["ms"],
        "fused_one_launch_ms": med["fused"]["ms"],
        "samples": med,
        "gemm_ms": ms_gemm,
        "quantize_ms": ms_quant,
        "quantize_gbs": (m * k * 2 + m * k + m * 4) / (ms_quant * 1e-3) / 1e9,
        "rotation256": {"ms_per_step": ms_step256, "tops": ops_count / (ms_step256 * 1e-3) / 1e12},
        "roofline": {
            "bound": "mfma", "achieved": gemm_tops, "peak": PEAK_INT8_TOPS, "unit": "TOPS",
            "frac": gemm_tops / PEAK_INT8_TOPS,
            "traffic": None if c2_traffic is None else c2_traffic["total"],
            "traffic_read_write": c2_traffic,
            "kernel": "gemm8_kernel (int8 256x256, 8 waves; bias+GELU epilogue)",
            "algorithmic_ops": ops_count, "algorithmic_bytes": traffic_alg,
        },
    }


def bench_c1(torch, ops, lib, stream) -> dict:
    """Config 1 on the GPU: M=128, K=N=3072, no rotation, per-token int8 (`cozyq_quantize_rot`
    with rotation 0) and the per-output-channel int8 weight, then the int8 GEMM (the narrow
    tiles at this M), bf16 out. 2.4 GOP: launch- and latency-bound, reported in µs and TOPS."""
    m, k, n = 128, 3072, 3072
    x = _activations(torch, m, k, 20261201)
    data, scale = ops.int8_quantize_rot(_weights(torch, n, k, 20261211), 0)
    q = torch.empty(m, k, dtype=torch.int8, device="cuda")
    s = torch.empty(m, dtype=torch.float32, device="cuda")
    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    xp, qp, sp, dp, wp, op = (t.data_ptr() for t in (x, q, s, data, scale, out))

    def quantize():
        _check(lib.cozyq_quantize_rot(0, xp, 0, qp, sp, m, k, 0, stream))

    def gemm():
        _check(lib.cozyq_gemm_ex(0, 0, qp, sp, dp, wp, None, op, n, 0, m, n, k, 0, stream))

    def step():
        quantize()
        gemm()

    preroll(torch, step)
    med = Timer(torch).interleaved({"step": step, "gemm": gemm, "quantize": quantize}, batch=16)
    ops_count = 2.0 * m * n * k
    return {"M": m, "K": k, "N": n, "us": med["step"]["ms"] * 1e3,
            "gemm_us": med["gemm"]["ms"] * 1e3, "quantize_us": med["quantize"]["ms"] * 1e3,
            "tops": ops_count / (med["step"]["ms"] * 1e-3) / 1e12,
            "kernel": "rotate_quantize_kernel (rotation 0) + narrow_kernel<int8>"}


def bench_decode(torch, ops, lib, stream, steps: int, warmup: int, m: int = 1) -> dict:
    """Config 3 at decode size: the fused fp8 linear (quantize + product in one launch: the GEMV
    to 4 rows, the row-tile kernel to 16), 8 rotating weight copies (470 MB, beyond the 256 MB
    MALL). A decode step is a few microseconds of GPU
    work, less than a Python-issued launch costs on the host, so the launches are captured
    once into a HIP graph (64 of them, 8 per copy) and the graph is replayed: `us` is GPU time
    per linear. `us_eager` is the same launches issued one by one from Python. The graph's
    output is checked bit for bit against an eager launch."""
    k, n, copies = 4096, 14336, 8
    x = _activations(torch, m, k, 31)
    weights = [ops.fp8_quantize(_weights(torch, n, k, 40 + c)) for c in range(copies)]
    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    ptrs = [(w.data_ptr(), s.data_ptr()) for w, s in weights]
    xp, op = x.data_ptr(), out.data_ptr()
    turn = [0]

    # Up to 16 rows: one fused launch (the GEMV to 4 rows, the row-tile kernel to 16). More
    # (or `two_launch`): quantize once, then the (narrow-tile) GEMM, the path
    # `Prebuilt.fp8_linear` takes past the fused kernels.
    q = torch.empty(m, k, dtype=torch.uint8, device="cuda")
    qs = torch.empty(m, dtype=torch.float32, device="cuda")

    def launch(raw_stream, fused=m <= 16):
        wp, sp = ptrs[turn[0] % copies]
        turn[0] += 1
        if fused:
            _check(lib.cozyq_fp8_linear(0, xp, 0, wp, sp, None, op, 0, m, n, k, raw_stream))
            return
        _check(lib.cozyq_quantize(0, 1, xp, 0, q.data_ptr(), qs.data_ptr(), m, k, None, None, 0,
                                  0, 1, 0, 0.0, 0, None, raw_stream))  # fmt: skip
        _check(lib.cozyq_gemm(0, 0, 1, q.data_ptr(), qs.data_ptr(), wp, sp, None, op, n, 0, m, n,
                              k, -1, None, None, raw_stream))  # fmt: skip

    eager_ms = Timer(torch).run(lambda: launch(stream), max(steps, 64), max(warmup, 8))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    per_graph = 8 * copies
    turn[0] = 0
    with torch.cuda.stream(side):
        launch(side.cuda_stream)  # warm the side stream
        torch.cuda.synchronize()
        turn[0] = 0
        with torch.cuda.graph(graph, stream=side):
            raw = torch.cuda.current_stream().cuda_stream
            for _ in range(per_graph):
                launch(raw)
    torch.cuda.synchronize()
    graph.replay()
    preroll(torch, graph.replay, 30)
    ms = Timer(torch).interleaved({"graph": graph.replay}, batch=2)["graph"]["ms"] / per_graph
    graph.replay()
    torch.cuda.synchronize()
    replayed = out.clone()
    turn[0] = copies - 1  # the graph's last launch used the last copy
    launch(stream)
    torch.cuda.synchronize()
    if not torch.equal(replayed, out):
        raise RuntimeError("decode: the graph replay differs from the eager launch")
    nbytes = n * k + n * 4 + m * k * 2 + m * n * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    row = {"M": m, "K": k, "N": n, "us": ms * 1e3, "us_eager": eager_ms * 1e3, "bytes": nbytes,
           "gbs": gbs, "frac": gbs / PEAK_HBM_GBS, "weight_copies": copies,
           "timing": "HIP graph of 64 launches, replayed; median of 15 samples of 2 replays"}
    if m <= 4:
        row["traffic"] = (pmc_traffic("decode", "void fp8_decode_kernel") or {}).get("total")
        row["kernel"] = "fp8_decode_kernel (quantize fused with the GEMV)"
    else:
        row["traffic"] = (pmc_traffic("fp8", "void fp8_rows_kernel") or {}).get("total")
        row["kernel"] = "fp8_rows_kernel (quantize fused with the row-tile product)"
        # The same graph-replayed timing of the two-launch path (quantize + narrow GEMM).
        row["us_quantize_then_gemm"] = _graph_us(
            torch, lambda raw: launch(raw, fused=False), 8 * copies, max(4, steps // 8))
    return row


def _graph_us(torch, launch, per_graph: int, replays: int) -> float:
    """GPU µs per launch of `launch(raw_stream)`, captured `per_graph` times into a HIP graph on a
    side stream and replayed."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        launch(side.cuda_stream)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            raw = torch.cuda.current_stream().cuda_stream
            for _ in range(per_graph):
                launch(raw)
    torch.cuda.synchronize()
    graph.replay()
    preroll(torch, graph.replay, 30)
    batch = max(1, min(4, replays // 4))
    return Timer(torch).interleaved({"graph": graph.replay}, batch=batch)["graph"]["ms"] / per_graph * 1e3


def _int8_decode_shape(torch, ops, lib, m: int, k: int, n: int, replays: int) -> dict:
    """The fused int8 GEMV (`cozyq_gemv`: rotation, quantization and GEMV in one launch) against
    the two-launch path (quantize, then the GEMM's shape rule: at 1..4 rows a GEMV on the codes)
    at one shape, each over enough rotating weight copies (> 600 MB) that the 256 MB MALL cannot
    hold them, graph-replayed; `int8_linear_takes` names the route `Prebuilt.int8_linear` takes."""
    copies = max(8, int(600e6 // (n * k)) + 1)
    x = _activations(torch, m, k, 61)
    weights = [ops.int8_quantize_rot(_weights(torch, n, k, 62 + c), 256) for c in range(copies)]
    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    q = torch.empty(m, k, dtype=torch.int8, device="cuda")
    qs = torch.empty(m, dtype=torch.float32, device="cuda")
    turn = [0]

    def fused(raw):
        w, ws = weights[turn[0] % copies]
        turn[0] += 1
        _check(lib.cozyq_gemv(0, x.data_ptr(), 0, w.data_ptr(), ws.data_ptr(), None, out.data_ptr(),
                              0, m, n, k, raw))  # fmt: skip

    def two_launch(raw):
        w, ws = weights[turn[0] % copies]
        turn[0] += 1
        _check(lib.cozyq_quantize(0, 0, x.data_ptr(), 0, q.data_ptr(), qs.data_ptr(), m, k, None,
                                  None, 0, 0, 1, 0, 0.0, 0, None, raw))  # fmt: skip
        _check(lib.cozyq_gemm(0, 0, 0, q.data_ptr(), qs.data_ptr(), w.data_ptr(), ws.data_ptr(),
                              None, out.data_ptr(), n, 0, m, n, k, -1, None, None, raw))  # fmt: skip

    us = _graph_us(torch, fused, 8 * copies if copies <= 8 else copies, replays)
    us_two = _graph_us(torch, two_launch, 8 * copies if copies <= 8 else copies, replays)
    nbytes = n * k + n * 4 + m * k * 2 + m * n * 2
    from cozyq import prebuilt

    return {"M": m, "K": k, "N": n, "us": us, "gbs": nbytes / (us * 1e-6) / 1e9,
            "frac_hbm": nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, "us_quantize_then_gemm": us_two,
            "weight_copies": copies,
            "int8_linear_takes": "one launch" if prebuilt.gemv_serves(m, k) else "quantize + GEMM"}


def bench_int8_decode(torch, ops, lib, stream, steps: int) -> dict:
    """The int8.convrot linear at decode size on config 2's weight (M=1, K=3072, N=12288), and
    the GEMV's wide rows (the reference's `gemv` range, `rotate.cu:453-468`: M=1 to K=32768, M=2
    to 16384, M=4 at an FFN-down's K=12288), each against quantize + GEMM."""
    replays = max(4, steps // 8)
    row = _int8_decode_shape(torch, ops, lib, 1, 3072, 12288, replays)
    row["kernel"] = "int8_decode_kernel (rotation + quantize fused with the GEMV)"
    row["wide_rows"] = [_int8_decode_shape(torch, ops, lib, m, k, n, replays)
                        for m, k, n in ((1, 32768, 4096), (2, 12288, 3072), (4, 12288, 3072))]
    return row


def bench_w4a8(torch, ops, lib, stream, steps: int) -> dict:
    """The w4a8.convrot GEMM on config 2's weight shape (K=3072, N=12288; 4-bit codes + E4M3
    group scales, 21.2 MB against int8's 37.7 MB) at M = 1 (the GEMV form), 16 and 32 (the row
    tile), 256 (the fused GEMM, codes unpacked in registers) and 4096 (unpack once + the 256x256
    int8 GEMM),
    int8.convrot's operand precomputed; bias + bf16 out; 14 rotating weight copies (297 MB,
    beyond the 256 MB MALL), one per call."""
    from cozyq import prebuilt

    k, n, copies = 3072, 12288, 14
    gen = torch.Generator(device="cuda").manual_seed(91)
    weights = []
    for _ in range(copies):
        codes = torch.randint(0, 256, (n, k // 2), generator=gen, device="cuda", dtype=torch.uint8)
        gs = (torch.randn(n, k // 16, generator=gen, device="cuda").abs() * 40 + 16).clamp(max=440)
        weights.append(prebuilt.W4a8(codes, gs.to(torch.float8_e4m3fn),
                                     (torch.rand(n, generator=gen, device="cuda") + 0.5) * 1e-3,
                                     None))  # fmt: skip
    bias = torch.randn(n, generator=gen, device="cuda").to(torch.bfloat16)
    levels = torch.empty(n, k, dtype=torch.int8, device="cuda")
    turn = [0]

    def next_weight():
        w = weights[turn[0] % copies]
        turn[0] += 1
        return w

    rows = []
    for m in (1, 16, 32, 256, 4096):
        q, s = ops.int8_quantize(_activations(torch, m, k, 92))
        out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
        args = (q.data_ptr(), s.data_ptr())

        def fused(st=stream):
            w = next_weight()
            _check(lib.cozyq_w4a8_gemm(0, *args, w.codes.data_ptr(), w.group_scale.data_ptr(),
                                       None, w.scale.data_ptr(), bias.data_ptr(), out.data_ptr(),
                                       0, m, n, k, -1, st))  # fmt: skip

        def unpacked():
            w = next_weight()
            _check(lib.cozyq_w4a8_unpack(0, w.codes.data_ptr(), w.group_scale.data_ptr(), None,
                                         levels.data_ptr(), n, k, stream))  # fmt: skip
            _check(lib.cozyq_gemm(0, 0, 0, *args, levels.data_ptr(), w.scale.data_ptr(),
                                  bias.data_ptr(), out.data_ptr(), n, 0, m, n, k, -1, None, None,
                                  stream))  # fmt: skip

        # Few rows: a HIP graph of launches, replayed (back-to-back launches from Python would
        # time the host's launch rate, not the kernel).
        if m < prebuilt.UNPACK_ROWS:
            ms = _graph_us(torch, fused, 2 * copies, steps) * 1e-3
        else:
            ms = Timer(torch).run(unpacked, steps, 5)
        weight_bytes = n * k // 2 + n * k // 16 + n * 4
        rows.append({"M": m, "us": ms * 1e3, "tops": 2.0 * m * n * k / (ms * 1e-3) / 1e12,
                     "weight_gbs": weight_bytes / (ms * 1e-3) / 1e9,
                     "path": ("GEMV (w4a8_decode_kernel)" if m <= 2 else "row-tile kernel (w4a8_rows_kernel)"
                              if m <= 32 else "fused narrow GEMM")
                     if m < prebuilt.UNPACK_ROWS else "unpack + int8 GEMM"})
    return {"K": k, "N": n, "rows": rows, "weight_copies": copies}


def bench_fp8(torch, ops, lib, stream, m: int, steps: int) -> dict:
    """Config 3's fp8 linear at M rows (K=4096, N=14336; per-token E4M3 activations, per-channel
    E4M3 weight) over 6 rotating weight copies (352 MB, beyond the 256 MB MALL), one per call:
    `us` the GEMM alone, `step_us` quantize + GEMM."""
    k, n, copies = 4096, 14336, 6
    x = _activations(torch, m, k, 33)
    weights = [ops.fp8_quantize(_weights(torch, n, k, 34 + c)) for c in range(copies)]
    q, s = ops.fp8_quantize(x)
    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    turn = [0]

    def gemm():
        data, scale = weights[turn[0] % copies]
        turn[0] += 1
        _check(lib.cozyq_gemm(0, 0, 1, q.data_ptr(), s.data_ptr(), data.data_ptr(),
                              scale.data_ptr(), None, out.data_ptr(), n, 0, m, n, k, -1, None,
                              None, stream))  # fmt: skip

    def step():
        _check(lib.cozyq_quantize(0, 1, x.data_ptr(), 0, q.data_ptr(), s.data_ptr(), m, k, None,
                                  None, 0, 0, 1, 0, 0.0, 0, None, stream))  # fmt: skip
        gemm()

    preroll(torch, step)
    med = Timer(torch).interleaved({"gemm": gemm, "step": step}, batch=max(2, min(8, steps // 4)))
    ms = med["gemm"]["ms"]
    tflops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    return {"M": m, "us": ms * 1e3, "step_us": med["step"]["ms"] * 1e3, "tflops": tflops,
            "frac_mfma": tflops / PEAK_FP8_TFLOPS, "weight_copies": copies}


def bench_mx(torch, ops, lib, stream, steps: int) -> dict:
    m = 4096
    shapes = {"qkv": (3072, 9216), "attn_out": (3072, 3072), "ffn_up": (3072, 12288),
              "ffn_down": (12288, 3072)}
    fns, sizes = {}, {}
    for name, (k, n) in shapes.items():
        x = _activations(torch, m, k, 71)
        data, wbyte = ops.mx_quantize(_weights(torch, n, k, 72))
        q = torch.empty(m, k, dtype=torch.float8_e4m3fn, device="cuda")
        qs = torch.empty(m, k // 32, dtype=torch.uint8, device="cuda")
        out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")

        def step(x=x, data=data, wbyte=wbyte, q=q, qs=qs, out=out, k=k, n=n):
            _check(lib.cozyq_mx_quantize(0, x.data_ptr(), 0, q.data_ptr(), qs.data_ptr(), m, k,
                                         stream))  # fmt: skip
            _check(lib.cozyq_mx_gemm(0, q.data_ptr(), qs.data_ptr(), data.data_ptr(),
                                     wbyte.data_ptr(), None, out.data_ptr(), n, 0, m, n, k,
                                     stream))  # fmt: skip

        fns[name], sizes[name] = step, (k, n)
    preroll(torch, lambda: [fn() for fn in fns.values()])
    med = Timer(torch).interleaved(fns, batch=max(2, min(8, steps // 4)))
    result, total_ops, total_ms = {}, 0.0, 0.0
    for name, (k, n) in sizes.items():
        ms = med[name]["ms"]
        ops_count = 2.0 * m * n * k
        total_ops += ops_count
        total_ms += ms
        result[name] = {"K": k, "N": n, "us": ms * 1e3, "tflops": ops_count / (ms * 1e-3) / 1e12}
    result["block_tflops"] = total_ops / (total_ms * 1e-3) / 1e12
    result["frac_mfma"] = result["block_tflops"] / PEAK_FP8_TFLOPS
    return result


def bench_svdq(torch, ops, lib, stream, steps: int) -> dict:
    """Config 4: SVDQuant W4A4 int4-g64, M=4096, K=N=3072, rank 32: the activation kernel
    (smoothing, int4 codes, la = bf16(x·downᵀ)) then the GEMM with the low-rank add and bias.
    The weight is the package encoder's (`cozyq.encode.encode_svdq_int4`) of W ~ N(0, 0.02)."""
    from cozyq import encode

    m, k, n, r = 4096, 3072, 3072, 32
    gen = torch.Generator().manual_seed(20261204)
    x = _activations(torch, m, k, 81)
    p = (torch.rand(k, generator=gen) * 1.5 + 0.5).cuda()
    down = (torch.randn(r, k, generator=gen) * 0.02).to(torch.bfloat16).cuda()
    up = (torch.randn(n, r, generator=gen) * 0.02).to(torch.bfloat16).cuda()
    encoded = encode.encode_svdq_int4(torch, "c4", (torch.randn(n, k, generator=gen) * 0.02).cuda(), p,
                                      down, up)  # fmt: skip
    codes, scales = encoded.payload, encoded.companions[0].raw
    bias = (torch.randn(n, generator=gen) * 0.5).to(torch.bfloat16).cuda()
    act = torch.empty(m, k // 2, dtype=torch.uint8, device="cuda")
    ascales = torch.empty(m, k // 64, dtype=torch.float16, device="cuda")
    la = torch.empty(m, r, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")

    def quantize():
        _check(lib.cozyq_svdq_int4_quantize(0, x.data_ptr(), 0, p.data_ptr(), down.data_ptr(),
                                            act.data_ptr(), ascales.data_ptr(), la.data_ptr(), m,
                                            k, r, stream))  # fmt: skip

    def gemm():
        _check(lib.cozyq_svdq_int4_gemm(0, act.data_ptr(), ascales.data_ptr(), codes.data_ptr(),
                                        scales.data_ptr(), la.data_ptr(), up.data_ptr(),
                                        bias.data_ptr(), out.data_ptr(), 0, m, n, k, r, stream))  # fmt: skip

    def step():
        quantize()
        gemm()

    preroll(torch, step)
    med = Timer(torch).interleaved({"quantize": quantize, "gemm": gemm, "step": step},
                                   batch=max(2, min(8, steps // 4)))  # fmt: skip
    q_ms, g_ms, ms = med["quantize"]["ms"], med["gemm"]["ms"], med["step"]["ms"]
    int4_ops = 2.0 * m * n * k
    lowrank_flops = 2.0 * m * r * (k + n)
    return {"M": m, "K": k, "N": n, "R": r, "us": ms * 1e3, "quantize_us": q_ms * 1e3,
            "gemm_us": g_ms * 1e3, "tops": (int4_ops + lowrank_flops) / (ms * 1e-3) / 1e12,
            "gemm_tops": int4_ops / (g_ms * 1e-3) / 1e12,
            "frac_int8_mfma": int4_ops / (g_ms * 1e-3) / 1e12 / PEAK_INT8_TOPS,
            "kernel": "svdq_gemm_kernel (int4 unpacked to int8, 32x32x32 MFMA, per-group rescale)"}


def bench_svdq_nvfp4(torch, ops, lib, stream, steps: int) -> dict:
    """Config 4's shape (M=4096, K=N=3072, rank 32) on the reference's own W4A4 law, svdq.nvfp4:
    g_x (`cozyq_svdq_input_scale`), the activation side (`cozyq_svdq_quantize`: nvfp4 codes and
    E4M3 scales of bf16(x·p), la = bf16(x·downᵀ)) and the GEMM (`cozyq_svdq_gemm`: both operands
    decoded exactly to fp16 on the MFMA, low-rank term and c in the epilogue, bias). The weight is
    random codes and scales in [0.5, ~3], as the reference's own probe draws it
    (`internal/svdq_linear.py:406-418`)."""
    m, k, n, r = 4096, 3072, 3072, 32
    gen = torch.Generator().manual_seed(20261205)
    x = _activations(torch, m, k, 82)
    roles = {
        "weight": torch.randint(0, 256, (n, k // 2), generator=gen).to(torch.uint8).cuda(),
        "scale": (torch.randn(n, k // 16, generator=gen).abs() + 0.5).to(torch.float8_e4m3fn).cuda(),
        "scale_2": torch.full((1,), 0.01).cuda(),
        "pre_quant_scale": (torch.rand(k, generator=gen) * 1.5 + 0.5).cuda(),
        "lowrank_down": (torch.randn(r, k, generator=gen) * 0.02).to(torch.bfloat16).cuda(),
        "lowrank_up": (torch.randn(n, r, generator=gen) * 0.02).to(torch.bfloat16).cuda(),
        "channel_scale": (torch.rand(n, generator=gen) + 0.5).cuda(),
    }
    bias = (torch.randn(n, generator=gen) * 0.5).to(torch.bfloat16).cuda()
    p = roles["pre_quant_scale"]
    g = ops.svdq_input_scale(x, p)
    act, ascales, la = ops.svdq_quantize(x, p, g, roles["lowrank_down"])

    def scale():
        ops.svdq_input_scale(x, p)

    def quantize():
        ops.svdq_quantize(x, p, g, roles["lowrank_down"])

    def gemm():
        ops.svdq_gemm(act, ascales, la, m, g, roles["weight"], roles["scale"], roles["scale_2"],
                      roles["lowrank_up"], roles["channel_scale"], bias, torch.bfloat16)  # fmt: skip

    def step():
        ops.svdq_linear(x, roles, bias, torch.bfloat16)

    preroll(torch, gemm)
    med = Timer(torch).interleaved({"scale": scale, "quantize": quantize, "gemm": gemm, "step": step},
                                   batch=max(2, min(8, steps // 4)))  # fmt: skip
    g_ms, ms = med["gemm"]["ms"], med["step"]["ms"]
    flops = 2.0 * m * n * k
    lowrank_flops = 2.0 * m * r * (k + n)
    return {"M": m, "K": k, "N": n, "R": r, "us": ms * 1e3, "input_scale_us": med["scale"]["ms"] * 1e3,
            "quantize_us": med["quantize"]["ms"] * 1e3, "gemm_us": g_ms * 1e3,
            "tflops": (flops + lowrank_flops) / (ms * 1e-3) / 1e12,
            "gemm_tflops": flops / (g_ms * 1e-3) / 1e12,
            "frac_f16_mfma": flops / (g_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
            "kernel": "nvfp4_gemm_kernel (E2M1 x E4M3 decoded to fp16, 32x32x16 f16 MFMA, 256x192 tiles by the round rule)"}


def bench_tiles(torch, ops, lib, stream, steps: int) -> dict:
    """The GEMM tile configs (`cozyq_gemm` config 0..5) at the shapes the shape rule
    (`cozyq_gemm_config`) was fitted on, int8 and fp8, as interleaved medians: each shape's per-
    config microseconds, the fastest config and the one config -1 runs."""
    from cozyq.prebuilt import GEMM_CONFIGS

    shapes = [(16, 14336, 4096), (64, 14336, 4096), (128, 14336, 4096), (128, 3072, 3072),
              (256, 14336, 4096), (256, 12288, 3072), (512, 14336, 4096), (1024, 14336, 4096),
              (4096, 14336, 4096), (4096, 12288, 3072), (4096, 9216, 3072), (4096, 3072, 3072),
              (4096, 3072, 12288), (8192, 640, 2560), (2048, 1280, 1280), (1024, 3072, 3072),
              (512, 3072, 3072), (2048, 3072, 3072), (16384, 3072, 3072), (384, 3072, 3072),
              (768, 3072, 3072), (4096, 1280, 5120), (1536, 3072, 3072), (64, 3072, 3072),
              (32, 12288, 3072)]  # fmt: skip
    configs = range(GEMM_CONFIGS)
    timer, rows = Timer(torch), []
    for kind in ("int8", "fp8"):
        for m, n, k in shapes:
            gen = torch.Generator(device="cuda").manual_seed(m + n + k)
            if kind == "int8":
                q = torch.randint(-127, 128, (m, k), dtype=torch.int8, device="cuda", generator=gen)
                w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda", generator=gen)
                f = ops.int8_gemm
            else:
                q = torch.randn(m, k, device="cuda", generator=gen).to(torch.float8_e4m3fn)
                w = (torch.randn(n, k, device="cuda", generator=gen) * 4).to(torch.float8_e4m3fn)
                f = ops.fp8_gemm
            xs = torch.rand(m, device="cuda", generator=gen) * 0.01 + 0.001
            ws = torch.rand(n, device="cuda", generator=gen) * 0.01 + 0.001
            bias = torch.randn(n, device="cuda", generator=gen).to(torch.bfloat16)
            fns = {c: (lambda c=c: f(q, xs, w, ws, bias, torch.bfloat16, c)) for c in configs}
            preroll(torch, fns[0], 30)
            est = timer.run(fns[0], 3, 1)
            med = timer.interleaved(fns, samples=9, batch=max(2, min(50, int(2.0 / max(est, 1e-3)))))
            us = {c: round(med[c]["ms"] * 1e3, 2) for c in configs}
            rows.append({"kind": kind, "M": m, "N": n, "K": k, "us": us, "best": min(us, key=us.get),
                         "chosen": lib.cozyq_gemm_config(int(kind == "fp8"), m, n, k)})  # fmt: skip
            del q, w
    return {"tiles": rows}


def bench_weights(torch, ops, lib, stream, steps: int) -> dict:
    """The stored-format decode kernels (checkpoint weight -> bf16) on the configs' weight
    shapes: int8.convrot (256) and mxfp8 (cuBLAS 128x4 scales) on config 2's [12288, 3072],
    fp8.rowwise on config 3's [14336, 4096], nvfp4 (high-first nibbles, 128x4 E4M3 scales,
    divide) on [12288, 3072] and svdq.nvfp4 (rank 32) on config 4's [3072, 3072]. Each runs over
    3 rotating (weight, destination) pairs (beyond the 256 MB MALL), graph-replayed through the
    C ABI. Bytes are the parts read once and the destination written once."""
    gen = torch.Generator(device="cuda").manual_seed(95)
    copies, replays = 3, max(4, steps // 8)

    def rnd(shape, dtype=torch.uint8):
        return torch.randint(0, 256, shape, generator=gen, device="cuda", dtype=torch.int32).to(torch.uint8).view(dtype)

    def measure(name, make, launch, nbytes):
        sets = [make() for _ in range(copies)]
        turn = [0]

        def go(raw):
            launch(sets[turn[0] % copies], raw)
            turn[0] += 1

        us = _graph_us(torch, go, 4 * copies, replays)
        return {"format": name, "us": us, "gbs": nbytes / (us * 1e-6) / 1e9,
                "frac_hbm": nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, "bytes": nbytes}

    out = []
    n, k = 12288, 3072

    def convrot():
        return (rnd((n, k), torch.int8), torch.rand(n, device="cuda"), torch.empty(n, k, dtype=torch.bfloat16, device="cuda"))

    out.append(measure("int8.convrot256 [12288,3072]", convrot, lambda t, raw: _check(lib.cozyq_decode_convrot(
        0, t[0].data_ptr(), t[1].data_ptr(), 0, 256, t[2].data_ptr(), 1, n, k, raw)), n * k * 3 + n * 4))

    n3, k3 = 14336, 4096

    def rowwise():
        return (rnd((n3, k3)), torch.rand(n3, device="cuda"), torch.empty(n3, k3, dtype=torch.bfloat16, device="cuda"))

    out.append(measure("fp8.rowwise [14336,4096]", rowwise, lambda t, raw: _check(lib.cozyq_decode(
        0, 1, t[0].data_ptr(), t[1].data_ptr(), 0, 1, 1, 0, None, 0, 0, None, 0, 0, 0, t[2].data_ptr(), 1,
        n3, k3, 1, raw)), n3 * k3 * 3 + n3 * 4))

    blocks = k // 32
    tiled = (-(-n // 128) * 128) * (-(-blocks // 4) * 4)

    def mx():
        return (rnd((n, k)) & 0x77, torch.randint(110, 130, (tiled,), device="cuda", dtype=torch.int32).to(torch.uint8),
                torch.empty(n, k, dtype=torch.bfloat16, device="cuda"))

    out.append(measure("mxfp8 128x4 [12288,3072]", mx, lambda t, raw: _check(lib.cozyq_decode(
        0, 1, t[0].data_ptr(), t[1].data_ptr(), 3, 3, 32, 1, None, 0, 0, None, 0, 0, 0, t[2].data_ptr(), 1,
        n, k, 1, raw)), n * k * 3 + tiled))

    tiled16 = (-(-n // 128) * 128) * (-(-(k // 16) // 4) * 4)
    second = torch.tensor([0.5], device="cuda")

    def nvfp4():
        return (rnd((n, k // 2)), rnd((tiled16,)) & 0x3F, torch.empty(n, k, dtype=torch.bfloat16, device="cuda"))

    out.append(measure("nvfp4 128x4 [12288,3072]", nvfp4, lambda t, raw: _check(lib.cozyq_decode(
        0, 3, t[0].data_ptr(), t[1].data_ptr(), 4, 3, 16, 1, second.data_ptr(), 0, 2, None, 0, 0, 1,
        t[2].data_ptr(), 1, n, k, 1, raw)), n * k // 2 + tiled16 + n * k * 2))

    n4, k4, rank = 3072, 3072, 32
    smooth = torch.rand(k4, device="cuda") + 0.5

    def svdq():
        return (rnd((n4, k4 // 2)), rnd((n4, k4 // 16)) & 0x3F,
                (torch.randn(rank, k4, device="cuda") * 0.05).to(torch.bfloat16),
                (torch.randn(n4, rank, device="cuda") * 0.05).to(torch.bfloat16),
                torch.empty(n4, k4, dtype=torch.bfloat16, device="cuda"))

    out.append(measure("svdq.nvfp4 r32 [3072,3072]", svdq, lambda t, raw: _check(lib.cozyq_decode_svdq(
        0, t[0].data_ptr(), t[1].data_ptr(), 0, 0, second.data_ptr(), 0, None, 0, smooth.data_ptr(), 0,
        t[2].data_ptr(), 1, t[3].data_ptr(), 1, rank, t[4].data_ptr(), 1, n4, k4, raw)),
        n4 * k4 // 2 + n4 * k4 // 16 + n4 * k4 * 2 + (n4 + k4) * rank * 2 + k4 * 4))
    return {"decode_formats": out}


def bench_nvfp4(torch, ops, lib, stream, steps: int) -> dict:
    """The nvfp4 W4A16 GEMV (`cozyq_nvfp4_gemv`) on config 3's weight shape (K=4096, N=14336:
    29.4 MB of E2M1 codes + 3.7 MB of tiled E4M3 scales, 0.56 bytes a weight) at M = 1 and 16,
    over 8 rotating weight copies (265 MB, beyond the MALL), graph-replayed; bf16 in and out. Then
    the routes past 16 rows against the reference's (`nvfp4_routes`)."""
    k, n, copies = 4096, 14336, 8
    gen = torch.Generator(device="cuda").manual_seed(97)
    tiled = (-(-n // 128) * 128) * (-(-(k // 16) // 4) * 4)
    weights = [(torch.randint(0, 256, (n, k // 2), generator=gen, device="cuda", dtype=torch.int32).to(torch.uint8),
                (torch.randint(0x30, 0x48, (tiled,), generator=gen, device="cuda", dtype=torch.int32)).to(torch.uint8))
               for _ in range(copies)]
    second = torch.tensor([0.02], device="cuda")
    out = []
    for m in (1, 16):
        x = _activations(torch, m, k, 98)
        y = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
        turn = [0]

        def go(raw):
            w, s = weights[turn[0] % copies]
            turn[0] += 1
            _check(lib.cozyq_nvfp4_gemv(0, x.data_ptr(), 0, w.data_ptr(), s.data_ptr(), second.data_ptr(),
                                        y.data_ptr(), 0, m, n, k, raw))  # fmt: skip

        us = _graph_us(torch, go, 8 * copies, max(4, steps // 8))
        nbytes = n * k // 2 + tiled + m * k * 2 + m * n * 2
        out.append({"M": m, "K": k, "N": n, "us": us, "gbs": nbytes / (us * 1e-6) / 1e9,
                    "frac_hbm": nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, "bytes": nbytes})
    return {"nvfp4_w4a16_gemv": out, "nvfp4_w4a16_routes": nvfp4_routes(torch, ops, weights[0], second, k, n)}


def nvfp4_routes(torch, ops, weight, second, k: int, n: int) -> list:
    """The nvfp4 leaf's routes past 16 rows against the reference's (decode the weight into x's
    dtype with scale_2 folded in, `cozyq_decode`, then the library GEMM,
    `internal/nvfp4_linear.py:376-385`): the GEMV at M = 32 and 48 on config 3's weight, and the
    one-launch W4A16 GEMM (`cozyq_nvfp4_gemm`) at 4096 x 12288 x 3072. Medians of 15
    interleaved samples."""
    from cozyq import decode as dec

    def rows(m, w, s, kk, nn):
        x = _activations(torch, m, kk, 99)
        decoded = torch.empty(nn, kk, dtype=torch.bfloat16, device="cuda")

        def reference():
            ops.decode_table(dec._CODE["u8"], w, s, dec._NUM["f8_e4m3fn"], decoded, nn, kk,
                             grid=dec.GRID_BLOCKS, block=16, tiled=True, scale_2=second)  # fmt: skip
            torch.nn.functional.linear(x, decoded)

        mine = (lambda: ops.nvfp4_gemv(x, w, s, second, torch.bfloat16)) if m <= 64 else \
            (lambda: ops.nvfp4_gemm(x, w, s, second, None, torch.bfloat16))
        preroll(torch, reference, 30)
        med = Timer(torch).interleaved({"cozyq": mine, "decode_blas": reference}, batch=8)
        kernel = "nvfp4_gemm_kernel<W4A16>" if m > 64 else (
            "nvfp4_rows_kernel" if m > 4 and kk % 128 == 0 and -(-nn // 64) >= 192 else "nvfp4_gemv_kernel")
        return {"M": m, "K": kk, "N": nn, "kernel": kernel,
                "us": med["cozyq"]["ms"] * 1e3, "decode_blas_us": med["decode_blas"]["ms"] * 1e3,
                "tflops": 2.0 * m * nn * kk / (med["cozyq"]["ms"] * 1e-3) / 1e12}

    out = [rows(m, weight[0], weight[1], k, n) for m in (32, 48)]
    gk, gn = 3072, 12288
    gen = torch.Generator(device="cuda").manual_seed(96)
    gw = torch.randint(0, 256, (gn, gk // 2), generator=gen, device="cuda", dtype=torch.int32).to(torch.uint8)
    gs = torch.randint(0x30, 0x48, (gn * gk // 16,), generator=gen, device="cuda", dtype=torch.int32).to(torch.uint8)
    out.append(rows(4096, gw, gs, gk, gn))
    return out


def bench_bake(torch, ops, lib, stream, steps: int) -> dict:
    """The LoRA bake (`cozyq_bake`, `cozyq_bake_nvfp4`) of a rank-32 update into config 2's
    weight shape ([12288, 3072]) in each stored form, in place, over 4 rotating weight copies,
    graph-replayed. Algorithmic bytes: the stored weight read and written, its scales, and the
    factors read once; the kernel's bound is the VALU (rank FMAs plus one Philox4x32-10 draw an
    element), which `gelems` (elements baked per second) reports."""
    from cozyq import bake as cb

    rows, cols, rank, copies = 12288, 3072, 32, 4
    gen = torch.Generator(device="cuda").manual_seed(131)
    up = torch.randn(rows, rank, generator=gen, device="cuda") * 1e-4
    down = torch.randn(rank, cols, generator=gen, device="cuda")
    rotated = cb.rotate_factor(torch, down)
    scale = torch.full((rows,), 0.01, device="cuda")
    second = torch.tensor([0.01], device="cuda")
    factors = 4 * rank * (rows + cols)
    forms = {
        "bf16": (cb.BF16, torch.bfloat16, 2 * rows * cols),
        "fp8.rowwise": (cb.ROWWISE, torch.uint8, rows * cols + 4 * rows),
        "int8.convrot": (cb.INT8, torch.int8, rows * cols + 4 * rows),
        "nvfp4": (cb.NVFP4, torch.uint8, rows * cols // 2 + rows * cols // 16),
    }
    out = []
    for name, (form, dtype, stored) in forms.items():
        if form == cb.NVFP4:
            weights = [(torch.randint(0, 256, (rows, cols // 2), generator=gen, device="cuda", dtype=torch.int32).to(torch.uint8),
                        torch.randint(0x30, 0x48, (rows, cols // 16), generator=gen, device="cuda", dtype=torch.int32).to(torch.uint8))
                       for _ in range(copies)]  # fmt: skip
        elif dtype == torch.bfloat16:
            weights = [(torch.randn(rows, cols, generator=gen, device="cuda") * 0.02).to(dtype) for _ in range(copies)]
        else:
            weights = [torch.randint(-100, 100, (rows, cols), generator=gen, device="cuda", dtype=torch.int32).to(dtype)
                       for _ in range(copies)]  # fmt: skip
        turn = [0]
        sides = rotated if form == cb.INT8 else down

        def go(raw, form=form, weights=weights, sides=sides):
            w = weights[turn[0] % copies]
            turn[0] += 1
            if form == cb.NVFP4:
                _check(lib.cozyq_bake_nvfp4(0, w[0].data_ptr(), w[1].data_ptr(), second.data_ptr(), up.data_ptr(),
                                            sides.data_ptr(), None, None, rows, cols, rank, 77, 0, raw))  # fmt: skip
            else:
                _check(lib.cozyq_bake(0, form, w.data_ptr(), scale.data_ptr(), up.data_ptr(), sides.data_ptr(),
                                      None, None, None, rows, cols, rank, 77, 0, raw))  # fmt: skip

        us = _graph_us(torch, go, 4 * copies, max(4, steps // 8))
        nbytes = 2 * stored + factors
        out.append({"form": name, "rows": rows, "cols": cols, "rank": rank, "us": us,
                    "gelems": rows * cols / (us * 1e-6) / 1e9, "gbs": nbytes / (us * 1e-6) / 1e9,
                    "frac_hbm": nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, "bytes": nbytes})
    return {"lora_bake": out}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as info:
            for line in info:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_threads() -> int:
    """The host threads the baseline uses: this process's CPU set, capped by OMP_NUM_THREADS
    where the job sets it (the GPU box gives one GPU's job a 16-thread share)."""
    cores = len(os.sched_getaffinity(0))
    cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return min(cores, cap) if cap > 0 else cores


def _cpu_seconds(fn, runs: int = 3) -> tuple[float, list[float]]:
    """One untimed warm-up call, then the median wall time of `runs` calls."""
    fn()
    times = []
    for _ in range(runs):
        start = time.perf_counter()
        fn()
        times.append(time.perf_counter() - start)
    return sorted(times)[len(times) // 2], times


def cpu_baselines(torch) -> dict:
    """The reference's CPU laws, restated in the oracle (`kind: "port"`), timed on this host's
    cores on a bounded sample of each config (one warm-up call, then the median of 3): C1 whole
    (rowwise int8, the literal int32 matmul), C2 on 1024 of its rows (rotation 128 + int8, int32
    matmul, scales, bias, GELU), C3 at M=1024 (e4m3 quantize, dequantize, float32 matmul: CPU
    torch's `_scaled_mm` rejects row-wise scales), C4 at M=1024 (int4-g64 quantize, dequantized
    float32 matmul + the bf16 low-rank branch; and the reference's svdq.nvfp4 `eager` law on the
    same shape), C5 on 512 rows of each DiT shape (MX quantize,
    E8M0 dequant, float32 matmul). `value` is the sample's ops per second."""
    from oracle import laws

    threads = _cpu_threads()
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(20261202)

    def acts(m, k):
        x = torch.randn(m, k, generator=gen)
        x[:, torch.randperm(k, generator=gen)[: k // 100]] *= 20
        return x.to(torch.bfloat16)

    def wts(n, k):
        return torch.randn(n, k, generator=gen) * 0.02

    bf16 = torch.bfloat16
    out = {}

    def record(name, fn, ops_count, unit, sample):
        seconds, times = _cpu_seconds(fn)
        out[name] = {"value": ops_count / seconds / 1e12, "unit": unit, "cores": threads,
                     "kind": "port", "seconds": seconds, "runs_s": times, "sample": sample}

    k1 = n1 = 3072
    x1 = acts(128, k1)
    d1, s1 = laws.int8_weight_rowwise(wts(n1, k1))
    record("c1", lambda: laws.int8_linear(x1, d1, s1, None, bf16, rotation=0, literal=True),
           2.0 * 128 * n1 * k1, "TOPS", "config 1 whole: X[128,3072] -> per-token int8, int32 "
           "matmul with W[3072,3072] rowwise int8, both scales, bf16")  # fmt: skip
    k2, n2, m2 = 3072, 12288, 1024
    x2 = acts(m2, k2)
    d2, s2 = laws.int8_weight_rotated(wts(n2, k2), 128)
    b2 = (torch.randn(n2, generator=gen) * 0.1).to(bf16)
    record("c2", lambda: laws.int8_linear(x2, d2, s2, b2, bf16, rotation=128, gelu=True, literal=True),
           2.0 * m2 * n2 * k2, "TOPS", f"config 2 rows 0..{m2 - 1}: X[{m2},{k2}] -> rotate(128)+int8, "
           f"int32 matmul with W[{n2},{k2}], scales, bias, tanh-GELU")  # fmt: skip
    k3, n3, m3 = 4096, 14336, 1024
    x3 = acts(m3, k3)
    d3, s3 = laws.fp8_weight(wts(n3, k3))
    record("c3", lambda: laws.fp8_linear(x3, d3, s3, None, bf16), 2.0 * m3 * n3 * k3, "TFLOPS",
           f"config 3 at M={m3}: e4m3 rowwise quantize, dequantize, float32 matmul with "
           f"W[{n3},{k3}] e4m3, bf16")  # fmt: skip
    k4 = n4 = 3072
    m4, r4 = 1024, 32
    x4 = acts(m4, k4)
    p4 = torch.rand(k4, generator=gen) * 1.5 + 0.5
    down4 = (torch.randn(r4, k4, generator=gen) * 0.02).to(bf16)
    up4 = (torch.randn(n4, r4, generator=gen) * 0.02).to(bf16)
    c4, sc4 = laws.svdq_weight(wts(n4, k4), p4, down4, up4)
    record("c4", lambda: laws.svdq_linear(x4, p4, c4, sc4, down4, up4, None, bf16),
           2.0 * m4 * n4 * k4 + 2.0 * m4 * r4 * (k4 + n4), "TOPS",
           f"config 4 at M={m4}: smoothing, int4-g64 quantize, dequantized float32 matmul with "
           f"W[{n4},{k4}] int4-g64, rank-32 bf16 low-rank branch")  # fmt: skip
    roles4 = {"weight": torch.randint(0, 256, (n4, k4 // 2), generator=gen).to(torch.uint8),
              "scale": (torch.randn(n4, k4 // 16, generator=gen).abs() + 0.5).to(torch.float8_e4m3fn),
              "scale_2": torch.full((1,), 0.01), "pre_quant_scale": p4, "lowrank_down": down4,
              "lowrank_up": up4}  # fmt: skip
    record("c4_nvfp4", lambda: laws.svdq_nvfp4_eager(x4, roles4, None, bf16),
           2.0 * m4 * n4 * k4 + 2.0 * m4 * r4 * (k4 + n4), "TFLOPS",
           f"config 4's shape at M={m4} on svdq.nvfp4 (internal/svdq_linear.py:639-659 `eager`): "
           f"g_x, nvfp4 fake-quantize, float32 matmul with the decoded W[{n4},{k4}], low-rank "
           "branch")  # fmt: skip
    m5 = 512
    mx_total_ops, mx_seconds = 0.0, 0.0
    for name, (k5, n5) in {"qkv": (3072, 9216), "attn_out": (3072, 3072), "ffn_up": (3072, 12288),
                           "ffn_down": (12288, 3072)}.items():  # fmt: skip
        x5 = acts(m5, k5)
        d5, e5 = laws.mx_quantize(wts(n5, k5))
        seconds, _ = _cpu_seconds(lambda: laws.mx_linear(x5, d5, e5, None, bf16))
        mx_total_ops += 2.0 * m5 * n5 * k5
        mx_seconds += seconds
    out["c5"] = {"value": mx_total_ops / mx_seconds / 1e12, "unit": "TFLOPS", "cores": threads,
                 "kind": "port", "seconds": mx_seconds,
                 "sample": f"config 5, {m5} rows through each of the four DiT shapes: MX quantize, "
                           "E8M0 dequant, float32 matmul"}
    cpu = _cpu_model()
    for entry in out.values():
        entry["cpu"] = cpu
    return out


def only(torch, ops, lib, stream, args) -> int:
    """One leg alone, for `rocprofv3` runs (kernel traces and counters per dispatch)."""
    if args.only == "copy":
        nbytes = 256 << 20
        src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        ms = Timer(torch).run(lambda: dst.copy_(src), args.steps, args.warmup)
        figures = {"copy_bytes": nbytes, "us": ms * 1e3, "gbs": 2 * nbytes / (ms * 1e-3) / 1e9}
    elif args.only == "c2":
        figures = bench_c2(torch, ops, lib, stream, args.steps, args.warmup, args.preroll_ms)
    elif args.only == "c1":
        figures = bench_c1(torch, ops, lib, stream)
    elif args.only == "decode":
        figures = bench_decode(torch, ops, lib, stream, args.steps, args.warmup)
    elif args.only == "fp8":
        figures = {"c3_fp8": [bench_fp8(torch, ops, lib, stream, m, args.steps) for m in (256, 4096)],
                   "c3_fp8_small": bench_decode(torch, ops, lib, stream, args.steps, args.warmup, m=16)}
    elif args.only == "mx":
        figures = bench_mx(torch, ops, lib, stream, args.steps)
    elif args.only == "int8_decode":
        figures = bench_int8_decode(torch, ops, lib, stream, args.steps)
    elif args.only == "w4a8":
        figures = bench_w4a8(torch, ops, lib, stream, args.steps)
    elif args.only == "weights":
        figures = bench_weights(torch, ops, lib, stream, args.steps)
    elif args.only == "nvfp4":
        figures = bench_nvfp4(torch, ops, lib, stream, args.steps)
    elif args.only == "bake":
        figures = bench_bake(torch, ops, lib, stream, args.steps)
    elif args.only == "svdq_nvfp4":
        figures = bench_svdq_nvfp4(torch, ops, lib, stream, args.steps)
    elif args.only == "tiles":
        figures = bench_tiles(torch, ops, lib, stream, args.steps)
    else:
        figures = bench_svdq(torch, ops, lib, stream, args.steps)
    print(json.dumps({"only": args.only, **figures}))
    return 0


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    # The chip's clocks settle over the first ~20 ms of sustained MFMA load (measured: the first
    # 20-launch round of the C2 GEMM runs ~12% slower than later ones), so the default warmup
    # covers that.
    parser.add_argument("--warmup", type=int, default=100)
    parser.add_argument("--preroll-ms", type=float, default=PREROLL_MS,
                        help="clock pre-roll before timing (profiling runs may shorten it)")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    parser.add_argument("--no-extra", action="store_true", help="skip configs 3-5")
    parser.add_argument("--only", choices=("c1", "c2", "decode", "int8_decode", "w4a8", "fp8", "svdq",
                                           "svdq_nvfp4", "mx", "weights", "nvfp4", "bake", "tiles",
                                           "copy"),
                        help="profiling aid: run one leg (or a plain 256 MiB device copy, the "
                             "counter calibration) --steps times and print its figures only")  # fmt: skip
    args = parser.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the linear shards "
              "along M with no exchange); run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    from cozyq import _lib, prebuilt

    ops = prebuilt.library(0)
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream

    if args.only:
        return only(torch, ops, lib, stream, args)
    c2 = bench_c2(torch, ops, lib, stream, args.steps, args.warmup, args.preroll_ms)
    print(f"[bench] c2 {c2['ms_per_step']:.4f} ms/step, gemm {c2['gemm_ms']:.4f} ms", file=sys.stderr, flush=True)
    decode = bench_decode(torch, ops, lib, stream, args.steps, args.warmup)
    print(f"[bench] decode M=1 {decode['us']:.2f} us {decode['gbs']:.0f} GB/s", file=sys.stderr, flush=True)
    configs = {}
    if not args.no_extra:
        configs["c1_int8_rowwise"] = [bench_c1(torch, ops, lib, stream)]
        configs["c3_fp8"] = [bench_fp8(torch, ops, lib, stream, m, max(10, args.steps // 2))
                             for m in (256, 4096)]  # fmt: skip
        configs["c3_fp8_small"] = [bench_decode(torch, ops, lib, stream, args.steps, args.warmup, m=16)]
        configs["int8_decode"] = bench_int8_decode(torch, ops, lib, stream, args.steps)
        configs["w4a8"] = bench_w4a8(torch, ops, lib, stream, max(10, args.steps // 2))
        configs["c4_svdq_w4a4"] = bench_svdq(torch, ops, lib, stream, max(10, args.steps // 2))
        configs["c4_svdq_nvfp4"] = bench_svdq_nvfp4(torch, ops, lib, stream, max(10, args.steps // 2))
        configs["c5_mxfp8"] = bench_mx(torch, ops, lib, stream, max(10, args.steps // 2))
        configs["weight_decode"] = bench_weights(torch, ops, lib, stream, args.steps)["decode_formats"]
        configs["nvfp4_w4a16"] = bench_nvfp4(torch, ops, lib, stream, args.steps)["nvfp4_w4a16_gemv"]
        configs["lora_bake"] = bench_bake(torch, ops, lib, stream, args.steps)["lora_bake"]
        print("[bench] extra configs done", file=sys.stderr, flush=True)
    baselines = None if args.no_cpu else cpu_baselines(torch)
    line = {
        "metric": METRIC,
        "value": c2["tops"],
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": c2["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "config 2: rotate(128)+per-token int8 + W8A8 int8 GEMM + bias + "
                               "tanh-GELU, bf16 out", "M": 4096, "K": 3072, "N": 12288,
                   "parallelism": "none (1 GPU)"},
        "roofline": c2["roofline"],
        "decode": decode,
        "preroll_ms": c2["preroll_ms"],
        "timing": f"value: {args.steps} steps between two synchronizations after {args.warmup} "
                  f"warm-up steps and a {PREROLL_MS:.0f} ms clock pre-roll; phase and config "
                  f"figures: medians of {SAMPLES} interleaved samples (HIP events)",
        "phases": {"quantize_ms": c2["quantize_ms"], "quantize_gbs": c2["quantize_gbs"],
                   "gemm_ms": c2["gemm_ms"], "step_median_ms": c2["step_median_ms"],
                   "samples": c2["samples"]},
        "configs": {"c2_rotation256": [c2["rotation256"]], **configs},
        "cpu_baseline": None if baselines is None else baselines["c2"],
        "cpu_baselines": baselines,
        "self_check": {name: v.detail for name, v in ops.verdicts.items()},
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())

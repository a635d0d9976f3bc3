"""Builds `cozyq/libcozyq.so` from `csrc/*.hip` for gfx950 with hipcc (no CMake, no torch).

    python cozy-runtime_amd/build.py [--verbose]

Each source compiles to an object under `_build/` in parallel, then one shared library is
linked. Every HIP compile carries `-ffp-contract=off` (the epilogues and quantizers round each
float32 step on its own, as the CPU law does) and disables packed-FP32 code generation.
"""

from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
SOURCES = ROOT / "csrc"
OBJECTS = ROOT / "_build"
LIBRARY = ROOT / "cozyq" / "libcozyq.so"
ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _compile(source: Path) -> Path:
    obj = OBJECTS / (source.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(source), "-o", str(obj)]
    done = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"
    lines = [ln for ln in (done.stdout + done.stderr).splitlines() if noise not in ln and ln.strip()]
    if done.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source.name}:\n" + "\n".join(lines))
    return obj


def build(verbose: bool = False) -> Path:
    """Compiles every source and links the library; returns its path."""
    OBJECTS.mkdir(exist_ok=True)
    sources = sorted(SOURCES.glob("*.hip"))
    workers = min(len(sources), max(1, (os.cpu_count() or 2) // 2), 8)
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = LIBRARY.with_suffix(".so.tmp")
    link = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    done = subprocess.run(link, capture_output=True, text=True)
    if done.returncode != 0:
        raise RuntimeError("link failed:\n" + done.stdout + done.stderr)
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY} from {len(sources)} sources", file=sys.stderr)
    return LIBRARY


if __name__ == "__main__":
    build(verbose="--verbose" in sys.argv)

"""Writes `philox_vectors.json`: Triton's `tl.randint` / `tl.rand` at a spread of seeds and uint32
offsets, from Triton's own CPU interpreter (`TRITON_INTERPRET=1`, the installed library; nothing
of the reference is imported). The bake's noise is these draws at counter `row * cols + col`, so
the vectors pin the oracle's seed/offset mapping and its uint → [0, 1) conversion.

Run here (no GPU needed): `TRITON_INTERPRET=1 python tests/golden/make_philox_vectors.py`.
"""

from __future__ import annotations

import json
import os
from pathlib import Path

os.environ.setdefault("TRITON_INTERPRET", "1")

import numpy as np  # noqa: E402
import torch  # noqa: E402
import triton  # noqa: E402
import triton.language as tl  # noqa: E402

SEEDS = [0, 1, 7, 12345, 0x2545F491, 0x7FFFFFFF]
N = 256


@triton.jit
def _draws(ints, floats, offsets, seed, N: tl.constexpr):
    o = tl.arange(0, N)
    at = tl.load(offsets + o).to(tl.uint32)
    tl.store(ints + o, tl.randint(seed, at))
    tl.store(floats + o, tl.rand(seed, at))


def main() -> None:
    rng = np.random.default_rng(20261201)
    picked = np.concatenate([
        np.arange(64), [0xFFFFFFFF, 0xFFFFFFFE, 0x80000000, 0x7FFFFFFF, 1 << 24, (1 << 24) + 1],
        rng.integers(0, 1 << 32, N - 70, dtype=np.int64),
    ]).astype(np.int64)  # fmt: skip
    cases = []
    for seed in SEEDS:
        ints = torch.zeros(N, dtype=torch.int32)
        floats = torch.zeros(N, dtype=torch.float32)
        offsets = torch.from_numpy(picked.astype(np.uint32).view(np.int32).copy())
        _draws[(1,)](ints, floats, offsets, seed, N)
        cases.append({
            "seed": seed,
            "offsets": [int(v) for v in picked],
            "randint": [int(v) & 0xFFFFFFFF for v in ints.tolist()],
            "rand_bits": [int(v) & 0xFFFFFFFF for v in floats.view(torch.int32).tolist()],
        })  # fmt: skip
    out = Path(__file__).with_name("philox_vectors.json")
    out.write_text(json.dumps({"triton": triton.__version__, "cases": cases}) + "\n")
    print(f"wrote {out} ({len(cases)} seeds x {N} offsets)")


if __name__ == "__main__":
    main()

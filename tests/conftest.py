"""Test setup: the package root on sys.path and the `gpu` marker.

`-m "not gpu"` runs the oracle checks, the host logic and the C-ABI load checks on the CPU;
`-m gpu` runs the parity tests of the HIP kernels against the oracle on an MI355X.
"""

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT, ROOT / "cozy-runtime_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")

"""CPU oracle for the quantized-linear hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the laws of cozy-runtime's quantized-linear path (activation
rotation, per-token int8 / fp8 quantization, MX block scaling, the W8A8 products) plus the two
laws this build defines where the reference has none (the 128-block rotation and the int4-g64
SVDQuant variant). It is the checker that the HIP kernels are compared against.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may import it, and
there only as the checker or as the timed CPU baseline — never as the thing measured for the GPU
and never as a fallback of the product path (`cozyq` never imports it).

Pins (how each law is checked against something other than itself) are listed per function in
`laws.py` and exercised by `tests/test_oracle.py`. Functions whose pin is weaker than a golden
vector or closed form say so in their docstring ("parity unpinned" where nothing pins them).
"""

from oracle import laws  # noqa: F401

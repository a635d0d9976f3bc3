"""cozyq: cozy-runtime's quantized-linear hot path, MI355X-native.

Hand-written HIP kernels for gfx950 (`csrc/`, built into `libcozyq.so` behind the C ABI of
`include/cozyq.h`) with a Python host layer that mirrors the reference's op surface:
`prebuilt.Prebuilt` (the op library), the per-format dispatchers `int8_linear`, `fp8_linear`,
`mx_linear` and `svdq_linear`, the operand-sharing API in `kernels`, and the encoded leaves and
their providers in `leaves` / `selection`.
"""

from cozyq._lib import KernelsAbsent  # noqa: F401

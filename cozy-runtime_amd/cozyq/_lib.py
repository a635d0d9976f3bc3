"""The C ABI of `include/cozyq.h`, loaded with ctypes: cozyq's stand-in for cozy-runtime's
`cozy_runtime._kernels._gemm` nanobind module (`kernels/csrc/gemm.cpp:194-222`).

The library is built in-tree (`cozy-runtime_amd/build.py`) next to this file. Loading it never
falls back to anything: a missing or unloadable library raises `KernelsAbsent` with the reason.
"""

from __future__ import annotations

import ctypes
from ctypes import c_double, c_float, c_int, c_int64, c_uint32, c_void_p
from pathlib import Path

PATH = Path(__file__).resolve().parent / "libcozyq.so"


class KernelsAbsent(RuntimeError):
    """The HIP library is not built or does not load here."""


_P = c_void_p
#: Every exported entry point and its (restype, argtypes).
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "cozyq_not_supported": (c_int, []),
    "cozyq_out_of_memory": (c_int, []),
    "cozyq_gemv_rows": (c_int, []),
    "cozyq_max_k": (c_int, []),
    "cozyq_arch": (ctypes.c_char_p, []),
    "cozyq_error_name": (ctypes.c_char_p, [c_int]),
    "cozyq_quantize": (
        c_int,
        [c_int, c_int, _P, c_int, _P, _P, c_int, c_int, _P, _P, c_int64, c_int64, c_int, c_int,
         c_float, c_int, _P, _P],
    ),
    "cozyq_quantize_rot": (c_int, [c_int, _P, c_int, _P, _P, c_int, c_int, c_int, _P]),
    "cozyq_w4a8_gemm": (c_int, [c_int, _P, _P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int,
                                c_int, _P]),
    "cozyq_w4a8_unpack": (c_int, [c_int, _P, _P, _P, _P, c_int, c_int, _P]),
    "cozyq_gemv": (c_int, [c_int, _P, c_int, _P, _P, _P, _P, c_int, c_int, c_int, c_int, _P]),
    "cozyq_gemm": (
        c_int,
        [c_int, c_int, c_int, _P, _P, _P, _P, _P, _P, c_int64, c_int, c_int, c_int, c_int, c_int,
         _P, _P, _P],
    ),
    "cozyq_gemm_config": (c_int, [c_int, c_int, c_int, c_int]),
    "cozyq_svdq_rows": (c_int, [c_int]),
    "cozyq_encode_svdq_int4": (
        c_int, [c_int, _P, c_int, _P, _P, _P, c_int, _P, _P, c_int64, c_int, _P]
    ),
    "cozyq_svdq_input_scale": (c_int, [c_int, _P, c_int, _P, c_int, c_int, _P, _P]),
    "cozyq_svdq_quantize": (
        c_int, [c_int, _P, c_int, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, _P]
    ),
    "cozyq_svdq_gemm": (
        c_int,
        [c_int, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, _P],
    ),
    "cozyq_linear_workspace_bytes": (c_int64, [c_int64]),
    "cozyq_linear_noalloc_max_rows": (c_int, []),
    "cozyq_linear_status": (c_int, [c_int, _P, _P]),
    "cozyq_linear_noalloc_status": (c_int, [c_int, _P]),
    "cozyq_linear_test_spin_limit": (None, [c_int]),
    "cozyq_linear_noalloc": (
        c_int,
        [c_int, _P, c_int, c_int, _P, _P, _P, _P, _P, _P, c_int64, c_int, c_int, c_int, c_int, c_int, _P],
    ),
    "cozyq_linear": (
        c_int,
        [c_int, _P, c_int, c_int, _P, _P, _P, _P, _P, _P, c_int64, c_int, c_int, c_int, c_int, c_int, _P, _P],
    ),
    "cozyq_gemm_ex": (
        c_int,
        [c_int, c_int, _P, _P, _P, _P, _P, _P, c_int64, c_int, c_int, c_int, c_int, c_int, _P],
    ),
    "cozyq_gemm_i32": (c_int, [c_int, _P, _P, _P, c_int, c_int, c_int, _P]),
    "cozyq_fp8_linear": (
        c_int, [c_int, _P, c_int, _P, _P, _P, _P, c_int, c_int, c_int, c_int, _P]
    ),
    "cozyq_mx_quantize": (c_int, [c_int, _P, c_int, _P, _P, c_int, c_int, _P]),
    "cozyq_mx_gemm": (
        c_int, [c_int, _P, _P, _P, _P, _P, _P, c_int64, c_int, c_int, c_int, c_int, _P]
    ),
    "cozyq_svdq_int4_quantize": (
        c_int, [c_int, _P, c_int, _P, _P, _P, _P, _P, c_int, c_int, c_int, _P]
    ),
    "cozyq_svdq_int4_gemm": (
        c_int,
        [c_int, _P, _P, _P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, _P],
    ),
    "cozyq_decode": (
        c_int,
        [c_int, c_int, _P, _P, c_int, c_int, c_int, c_int, _P, c_int, c_int, _P, c_int, c_int,
         c_int, _P, c_int, c_int64, c_int64, c_int, _P],
    ),
    "cozyq_decode_convrot": (
        c_int, [c_int, _P, _P, c_int, c_int, _P, c_int, c_int64, c_int64, _P]
    ),
    "cozyq_decode_svdq": (
        c_int,
        [c_int, _P, _P, c_int, c_int, _P, c_int, _P, c_int, _P, c_int, _P, c_int, _P, c_int,
         c_int, _P, c_int, c_int64, c_int64, _P],
    ),
    "cozyq_nvfp4_gemv": (c_int, [c_int, _P, c_int, _P, _P, _P, _P, c_int, c_int, c_int, c_int, _P]),
    "cozyq_nvfp4_gemm": (c_int, [c_int, _P, c_int, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, _P]),
    "cozyq_encode_int8_convrot": (c_int, [c_int, _P, c_int, _P, _P, c_int64, c_int, _P]),
    "cozyq_encode_w4a8": (c_int, [c_int, _P, c_int, _P, _P, _P, _P, c_int64, c_int, _P]),
    "cozyq_encode_fp8_rowwise": (c_int, [c_int, _P, c_int, _P, _P, c_int64, c_int, _P]),
    "cozyq_encode_mxfp8": (c_int, [c_int, _P, c_int, _P, _P, c_int, c_int64, c_int, _P]),
    "cozyq_encode_nvfp4": (
        c_int, [c_int, _P, c_int, _P, _P, _P, _P, _P, c_int64, c_int, _P]
    ),
    "cozyq_measure": (c_int, [c_int, _P, c_int, _P, c_int64, _P, c_int, _P, _P]),
    "cozyq_bake": (
        c_int, [c_int, c_int, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_uint32, c_int, _P]
    ),
    "cozyq_bake_nvfp4": (
        c_int, [c_int, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_uint32, c_int, _P]
    ),
    "cozyq_bake_norms": (
        c_int, [c_int, c_int, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, _P, _P]
    ),
    "cozyq_bake_nvfp4_refit": (
        c_int, [c_int, _P, _P, _P, c_double, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_uint32, c_int, _P]
    ),
    "cozyq_bake_feedback": (c_int, [c_int, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, _P]),
    "cozyq_bake_stats": (
        c_int, [c_int, c_int, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, _P, _P]
    ),
    "cozyq_bake_row_amax": (
        c_int, [c_int, c_int, _P, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, _P, _P]
    ),
    "cozyq_bake_rotate_factor": (c_int, [c_int, _P, _P, c_int64, c_int64, _P]),
    "cozyq_host_e4m3": (None, [_P, _P, c_int64]),
    "cozyq_host_mx_byte": (None, [_P, _P, c_int64]),
    "cozyq_probe_div": (c_int, [c_int, _P, _P, _P, c_int64, _P]),
    "cozyq_probe_e4m3": (c_int, [c_int, _P, _P, c_int64, _P]),
    "cozyq_probe_e2m1": (c_int, [c_int, _P, _P, c_int64, _P]),
    "cozyq_probe_mfma": (c_int, [c_int, c_int, _P, _P, _P, _P, _P, _P]),
}

_LIB: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """The library with every signature declared; raises `KernelsAbsent` when it cannot load."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not PATH.exists():
        raise KernelsAbsent(f"{PATH} is not built: run `python cozy-runtime_amd/build.py`")
    try:
        lib = ctypes.CDLL(str(PATH))
    except OSError as exc:
        raise KernelsAbsent(f"{PATH} does not load: {exc}") from exc
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _LIB = lib
    return lib


def error_name(code: int) -> str:
    return load().cozyq_error_name(code).decode()

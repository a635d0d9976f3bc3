"""The C-ABI library on the CPU: it loads, exports every entry point `include/cozyq.h` declares
(and ctypes binds each), and the kernels' scalar conversions — compiled for the host from the
same source — agree with torch's casts and the oracle's exponent law. No GPU call is made."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import torch

from cozyq import _lib
from oracle import laws

HEADER = Path(__file__).resolve().parents[1] / "include" / "cozyq.h"


def _declared() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"\b(cozyq_[a-z0-9_]+)\s*\(", text)) - {"cozyq_allocate_fn"}


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(lib, name), name
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)


def test_constants():
    lib = _lib.load()
    assert lib.cozyq_not_supported() == 801  # hipErrorNotSupported
    assert lib.cozyq_out_of_memory() == 2  # hipErrorOutOfMemory
    assert lib.cozyq_gemv_rows() == 4
    assert lib.cozyq_max_k() == 32768
    assert lib.cozyq_arch() == b"gfx950"
    assert _lib.error_name(801) == "hipErrorNotSupported"


def test_gemm_config_rule():
    """`cozyq_gemm_config` (what config -1 runs): from 160 256x256 tiles a 256-row tile, the
    256x192 one (5) where its grid needs fewer than 6/5 the rounds of 256x256 tiles over the 256
    CUs (a round of 3/4-size tiles at ~90% of the rate), else 256x256 (0);
    else, when N gives a 64-column tile 192 workgroups, the one (4: 32x64, 3: 64x64, 2: 128x64)
    that takes every row (up to 128) in one M-tile; else the largest of 1: 128x128, 2: 128x64,
    3: 64x64, 4: 32x64 whose grid reaches 288 workgroups, else 32x64. Each case below is the
    fastest config the MI355X sweep (`bench.py --only tiles`) measured within 3% at that shape,
    for int8 and fp8 alike, except (8192, 640, 2560), where 128x64 is 8% faster."""
    lib = _lib.load()
    cases = {(4096, 12288, 3072): 0, (4096, 3072, 3072): 5, (1024, 14336, 4096): 0,
             (16384, 3072, 3072): 0, (4096, 3072, 12288): 5, (2048, 3072, 3072): 1,
             (4096, 9216, 3072): 5, (4096, 14336, 4096): 0,
             (1024, 3072, 3072): 2, (768, 3072, 3072): 2, (512, 3072, 3072): 3,
             (384, 3072, 3072): 3, (1536, 3072, 3072): 1, (512, 14336, 4096): 1,
             (256, 14336, 4096): 2, (256, 12288, 3072): 2, (2048, 1280, 1280): 2,
             (4096, 1280, 5120): 1, (8192, 640, 2560): 1, (16, 14336, 4096): 4,
             (1, 14336, 4096): 4, (64, 14336, 4096): 3, (128, 14336, 4096): 2,
             (128, 3072, 3072): 4, (64, 3072, 3072): 4, (32, 12288, 3072): 4}  # fmt: skip
    for (m, n, k), want in cases.items():
        for fp8 in (0, 1):
            assert lib.cozyq_gemm_config(fp8, m, n, k) == want, (m, n, k, fp8)
    assert lib.cozyq_gemm_config(0, 0, 8, 256) == -1


def test_nvfp4_entry_points_refuse_bad_shapes_before_the_device():
    """`cozyq_nvfp4_gemv` takes 0..64 rows and K % 32 == 0; `cozyq_nvfp4_gemm` K % 64 == 0 and
    N % 8 == 0. Refusals (hipErrorInvalidValue = 1) and the empty product come back before any
    device call."""
    lib = _lib.load()
    buf = ctypes.create_string_buffer(4096 + 16)
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16
    g = ctypes.c_void_p(p)
    assert lib.cozyq_nvfp4_gemv(0, p, 0, p, p, g, p, 0, 65, 64, 64, None) == 1
    assert lib.cozyq_nvfp4_gemv(0, p, 0, p, p, g, p, 0, 4, 64, 48, None) == 1
    assert lib.cozyq_nvfp4_gemv(0, None, 0, p, p, g, None, 0, 0, 64, 64, None) == 0
    assert lib.cozyq_nvfp4_gemm(0, p, 0, p, p, g, None, p, 0, 300, 64, 96, None) == 1
    assert lib.cozyq_nvfp4_gemm(0, p, 0, p, p, g, None, p, 0, 300, 60, 64, None) == 1
    assert lib.cozyq_nvfp4_gemm(0, p, 0, p, p, g, None, p + 8, 0, 300, 64, 64, None) == 1
    assert lib.cozyq_nvfp4_gemm(0, None, 0, p, p, g, None, None, 0, 0, 64, 64, None) == 0


def _host(fn: str, values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, dtype=np.float32)
    out = np.zeros(values.shape, dtype=np.uint8)
    getattr(_lib.load(), fn)(values.ctypes.data_as(ctypes.c_void_p),
                             out.ctypes.data_as(ctypes.c_void_p), values.size)  # fmt: skip
    return out


def _every(dtype: torch.dtype) -> np.ndarray:
    raw = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(dtype).float()
    return raw[torch.isfinite(raw)].numpy()


def test_device_e4m3_encoder_matches_torch_cast():
    """The kernels' `e4m3_rn` against `.to(float8_e4m3fn)` on every bf16 and fp16 value in
    range, on float32 values at and beside every E4M3 rounding midpoint, and on random float32."""
    gen = np.random.default_rng(0)
    v = np.concatenate([_every(torch.bfloat16), _every(torch.float16),
                        gen.standard_normal(200000).astype(np.float32) * 100])  # fmt: skip
    codes = np.arange(0, 0x7F, dtype=np.uint8)
    vals = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    bits = mids.view(np.uint32)
    v = np.concatenate([v, mids, (bits + 1).view(np.float32), (bits - 1).view(np.float32)])
    v = np.concatenate([v, -v])
    v = v[np.abs(v) <= 448]
    got = _host("cozyq_host_e4m3", v)
    want = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, want)


def test_device_mx_byte_matches_the_law():
    """The kernels' `mx_byte` against the law's torch log2/ceil for every positive bf16/fp16
    block maximum, zero and the extremes."""
    for dtype in (torch.bfloat16, torch.float16):
        v = _every(dtype)
        v = np.concatenate([v[v > 0], [0.0]]).astype(np.float32)
        block = torch.zeros(v.size, 32)
        block[:, 0] = torch.from_numpy(v)
        _, want = laws.mx_quantize(block.to(dtype))
        assert np.array_equal(_host("cozyq_host_mx_byte", v), want.reshape(-1).numpy())

"""GPU parity of the fused int8 linear (`cozyq_linear`: rotation, per-token int8 and the GEMM
with its epilogue in one persistent launch) against the CPU law and the two-launch path.

Bar: the operand (codes, scales) and the outputs bit-exact to `oracle/laws.py` (the int8 law of
`internal/int8_linear.py:415-448` + `:276`); the tanh-GELU epilogue bit-exact to the two-launch
GEMM's (the same epilogue code), which the GELU tests hold to the float64 law.
"""

from __future__ import annotations

import pytest
import torch

from fullsize import tile_rows
from oracle import laws

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def ops():
    from cozyq import prebuilt

    return prebuilt.library(0)


def activations(m: int, k: int, seed: int, dtype=torch.bfloat16) -> torch.Tensor:
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=gen)
    x[:, torch.randperm(k, generator=gen)[: max(1, k // 100)]] *= 20
    return x.to(dtype)


def weight(n: int, k: int, rotation: int, seed: int):
    w = torch.randn(n, k, generator=torch.Generator().manual_seed(seed)) * 0.02
    return laws.int8_weight_rotated(w, rotation) if rotation else laws.int8_weight_rowwise(w)


#: (M, N, K): one M-tile, ragged rows, 10 M-tiles (queues owning a pair and a single), K at the
#: one-wave limit, N not a multiple of the tile.
SHAPES = [(1, 264, 1024), (100, 264, 768), (257, 520, 1024), (2309, 264, 2048), (600, 1032, 4096)]


@pytest.mark.parametrize("bias", [False, True], ids=["nobias", "bias"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("rotation", [256, 128, 0])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_fused_linear_bit_exact(ops, shape, rotation, dtype, bias):
    m, n, k = shape
    if rotation and k % rotation:
        pytest.skip("K is a multiple of the rotation")
    x = activations(m, k, seed=m + n + k + rotation, dtype=dtype)
    x[m // 2] = 0  # the scale floor
    data, scale = weight(n, k, rotation, seed=n + k)
    b = (torch.randn(n, generator=torch.Generator().manual_seed(3)) * 0.1).to(dtype) if bias else None
    got = ops.int8_linear_rot(x.to(DEV), data.to(DEV), scale.to(DEV), None if b is None else b.to(DEV),
                              dtype, rotation)  # fmt: skip
    assert got is not None
    out, q, s = got
    wq, ws = laws.quantize_rows_int8(x, rotation)
    assert torch.equal(q.cpu(), wq)
    assert torch.equal(s.cpu().view(torch.int32), ws.reshape(-1).view(torch.int32))
    assert torch.equal(out.cpu(), laws.int8_linear(x, data, scale, b, dtype, rotation=rotation))


@pytest.mark.parametrize("rotation", [256, 128])
def test_fused_gelu_equals_two_launch(ops, rotation):
    """The tanh-GELU epilogue: bit for bit what quantize + `cozyq_gemm_ex` write (the same
    epilogue code); both held to the float64 law by `test_int8_gemm_rotation_lanes_and_gelu`."""
    m, n, k = 1100, 520, 3072
    x = activations(m, k, seed=5).to(DEV)
    data, scale = weight(n, k, rotation, seed=6)
    data, scale = data.to(DEV), scale.to(DEV)
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(7)) * 0.1).to(torch.bfloat16).to(DEV)
    out, q, s = ops.int8_linear_rot(x, data, scale, bias, torch.bfloat16, rotation, 1)
    q2, s2 = ops.int8_quantize_rot(x, rotation)
    two = ops.int8_gemm_ex(q2, s2, data, scale, bias, torch.bfloat16, 1)
    assert torch.equal(q, q2) and torch.equal(s, s2)
    assert torch.equal(out, two)


def test_fused_linear_calls_in_a_row_leave_the_workspace_zero(ops):
    """Calls in stream order share one workspace: each leaves its counters zero, so a larger
    call, then a smaller one, then a larger one again, all equal the law."""
    k, n = 1024, 264
    data, scale = weight(n, k, 256, seed=9)
    data, scale = data.to(DEV), scale.to(DEV)
    for m in (3000, 40, 2600):
        x = activations(m, k, seed=m)
        out, _, _ = ops.int8_linear_rot(x.to(DEV), data, scale, None, torch.bfloat16, 256)
        assert torch.equal(out.cpu(), laws.int8_linear(x, data.cpu(), scale.cpu(), None, torch.bfloat16))
    torch.cuda.synchronize()
    for work in ops._workspaces.values():
        assert not work.any()


def test_fused_linear_declines(ops):
    """Rows past 4096 elements, or an output dtype other than x's, answer NOT_SUPPORTED
    (None here) and `int8_linear` then quantizes + multiplies: still the law."""
    n = 264
    data, scale = weight(n, 4352, 256, seed=11)
    x = activations(50, 4352, seed=12)
    assert ops.int8_linear_rot(x.to(DEV), data.to(DEV), scale.to(DEV), None, torch.bfloat16, 256) is None
    got = ops.int8_linear(x.to(DEV), data.to(DEV), scale.to(DEV), None, torch.bfloat16)
    assert torch.equal(got.cpu(), laws.int8_linear(x, data, scale, None, torch.bfloat16))
    data, scale = weight(n, 1024, 256, seed=13)
    x = activations(50, 1024, seed=14)
    assert ops.int8_linear_rot(x.to(DEV), data.to(DEV), scale.to(DEV), None, torch.float16, 256) is None


def test_c2_full_size_fused_equals_two_launch(ops):
    """BASELINE config 2 at its real shape through the fused launch: every code and scale of the
    operand bit-exact to the CPU law; the bias + GELU outputs of 4 rows of every M-tile (each
    against every column) within tolerance of the float64 law; and the whole output bit-exact to
    the two-launch path's."""
    m, k, n = 4096, 3072, 12288
    x = activations(m, k, seed=20261202)
    data, scale = weight(n, k, 128, seed=20261203)
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(5)) * 0.1).to(torch.bfloat16)
    dd, ds, db = data.to(DEV), scale.to(DEV), bias.to(DEV)
    out, q, s = ops.int8_linear_rot(x.to(DEV), dd, ds, db, torch.bfloat16, 128, 1)
    wq, ws = laws.quantize_rows_int8(x, 128)
    assert torch.equal(q.cpu(), wq)
    assert torch.equal(s.cpu().view(torch.int32), ws.reshape(-1).view(torch.int32))
    rows = tile_rows(m)
    exact = laws.int32_gemm(wq[rows], data).double() * ws[rows].double() * scale.double()
    exact = laws.gelu_tanh((exact + bias.double()).float()).double()
    got = out.cpu()[rows].double()
    rms = exact.pow(2).mean().sqrt()
    assert ((got - exact).abs() <= 1e-2 * rms + 2e-2 * exact.abs()).all()
    q2, s2 = ops.int8_quantize_rot(x.to(DEV), 128)
    assert torch.equal(out, ops.int8_gemm_ex(q2, s2, dd, ds, db, torch.bfloat16, 1))


def test_fused_linear_reports_a_wait_that_gives_up(ops):
    """The bounded wait's failure path, forced from the host (`cozyq_linear_test_spin_limit(-1)`
    makes every workgroup give up before it waits, so every kernel exits normally): every output
    is the output dtype's NaN, never a tile computed from codes that may not exist yet; the status
    read reports it once and clears it; the quantize jobs still write the law's operand; the
    counters are left zero, and the next call, at the default limit, is the law again."""
    lib = ops._lib
    m, n, k = 600, 520, 1024
    x = activations(m, k, seed=31)
    data, scale = weight(n, k, 256, seed=32)
    dx, dd, ds = x.to(DEV), data.to(DEV), scale.to(DEV)
    lib.cozyq_linear_test_spin_limit(-1)
    try:
        for dtype in (torch.bfloat16, torch.float16):
            out, q, s = ops.int8_linear_rot(dx.to(dtype), dd, ds, None, dtype, 256)
            torch.cuda.synchronize()
            assert torch.isnan(out.cpu().float()).all()
            wq, ws = laws.quantize_rows_int8(x.to(dtype), 256)
            assert torch.equal(q.cpu(), wq)
            assert torch.equal(s.cpu().view(torch.int32), ws.reshape(-1).view(torch.int32))
    finally:
        lib.cozyq_linear_test_spin_limit(0)
    with pytest.raises(RuntimeError, match="gave up"):
        ops.linear_status()
    ops.linear_status()  # the record was cleared by the read
    for work in ops._workspaces.values():
        assert not work.any()
    out, _, _ = ops.int8_linear_rot(dx, dd, ds, None, torch.bfloat16, 256, verify=True)
    assert torch.equal(out.cpu(), laws.int8_linear(x, data, scale, None, torch.bfloat16))

"""The op library's argument contract (V1-V6) and the svdq low-rank helpers (R1-R3), on the
CPU: each single violation raises the reference's message (`internal/prebuilt.py:360-406`,
`:193-250`, `:263-291`), and the admission table reports faults in its fixed order. The
library loads here (no GPU call is made)."""

from __future__ import annotations

import pytest
import torch

from cozyq import _admit, prebuilt, svdq_linear


@pytest.fixture(scope="module")
def ops():
    return prebuilt.Prebuilt(torch, 0)


def _aligned_empty(*shape, dtype):
    """A tensor at a 16-byte address (a slice of a larger byte buffer where needed)."""
    n = 1
    for d in shape:
        n *= d
    size = n * torch.empty(0, dtype=dtype).element_size()
    raw = torch.zeros(size + 16, dtype=torch.uint8)
    skip = (-raw.data_ptr()) % 16
    return raw[skip:skip + size].view(dtype).view(*shape)


def test_faults_in_fixed_order():
    spec = _admit.Operand(kinds=(torch.int8,), extents=(None, 64), dense=True, align=16, rows=8)
    t = _aligned_empty(12, 128, dtype=torch.int8)[:, ::2]  # 64 wide, strided, 12 rows
    assert _admit.faults(t, spec) == [_admit.LAYOUT, _admit.ROWS]
    assert _admit.faults(torch.zeros(16, 64, dtype=torch.int8), spec) in ([], [_admit.ALIGN])
    assert _admit.faults(torch.zeros(16, 65, dtype=torch.float32), spec)[:2] == [_admit.KIND, _admit.EXTENT]
    assert _admit.faults(torch.zeros(3), _admit.Operand(count=4)) == [_admit.EXTENT]


def test_placement_takes_only_in_place_layouts():
    place = _admit.Placement(4, 8, torch.bfloat16, torch.device("cpu"))
    wide = _aligned_empty(4, 16, dtype=torch.bfloat16)
    assert place.takes(_aligned_empty(4, 8, dtype=torch.bfloat16))
    assert not place.takes(torch.zeros(4, 8, dtype=torch.float16))
    assert not place.takes(torch.zeros(8, 4, dtype=torch.bfloat16).t())
    assert place.takes(wide[:, :8])  # rows 32 bytes apart: written in place
    assert not place.takes(torch.zeros(4, 12, dtype=torch.bfloat16)[:, :8])  # rows 24 bytes apart


def test_weight_messages(ops):
    f = prebuilt.INT8
    data = _aligned_empty(64, 256, dtype=torch.int8)
    scale = torch.ones(64)
    cases = [
        (data.float(), scale, "int8: data must be torch.int8 [N, 256]"),
        (data[:, :128], scale, "int8: data must be torch.int8 [N, 256]"),
        (_aligned_empty(60, 256, dtype=torch.int8), torch.ones(60), "data must be contiguous, aligned, N a multiple of 8"),
        (torch.empty(256, 64, dtype=torch.int8).t(), scale, "data must be contiguous, aligned, N a multiple of 8"),
        (data, torch.ones(63), "int8: scale must be float32 with 64 values"),
        (data, torch.ones(64, dtype=torch.float64), "int8: scale must be float32 with 64 values"),
        (data, torch.ones(128)[::2], "int8: scale must be contiguous"),
        (data, scale, "int8: the weight's tensors must be on cuda:0"),
    ]
    for d, s, text in cases:
        with pytest.raises(ValueError, match=text.replace("[", r"\[").replace("]", r"\]")):
            ops._weight(f, d, s, None, 256, torch.bfloat16)


def test_operand_and_rows_messages(ops):
    q = _aligned_empty(8, 256, dtype=torch.int8)
    with pytest.raises(ValueError, match=r"int8_gemm: q must be a contiguous, aligned torch.int8 \[M, K\]"):
        ops._operand("int8_gemm", torch.int8, q.float(), torch.ones(8))
    with pytest.raises(ValueError, match="int8_gemm: scales must be contiguous float32 with 8 values"):
        ops._operand("int8_gemm", torch.int8, q, torch.ones(7))
    assert ops._operand("int8_gemm", torch.int8, q, torch.ones(8)) == (8, 256)
    with pytest.raises(ValueError, match="int8: x must be on cuda:0"):
        ops._rows(prebuilt.INT8, torch.zeros(2, 256, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="bf16 or fp16, not torch.float32"):
        ops._half(torch.float32)
    assert ops._half(torch.float16) is True and ops._half(torch.bfloat16) is False


def test_w4a8_weight_messages(ops):
    n, k = 16, 256

    def weight(**over):
        base = {"codes": _aligned_empty(n, k // 2, dtype=torch.uint8),
                "group_scale": torch.ones(n, k // 16).to(torch.float8_e4m3fn),
                "scale": torch.ones(n), "codebook": None}  # fmt: skip
        base.update(over)
        return prebuilt.W4a8(**base)

    shapes = r"w4a8: codes, group scales and scale must be \[16, 128\], \[16, 16\] and \[16\], contiguous"
    cases = [
        (weight(codes=_aligned_empty(n, k // 4, dtype=torch.uint8)), shapes),
        (weight(scale=torch.ones(n + 1)), shapes),
        (weight(codes=_aligned_empty(n, k // 4, dtype=torch.int16)), "w4a8: codes are bytes and group scales E4M3"),
        (weight(group_scale=torch.ones(n, k // 16)), "w4a8: codes are bytes and group scales E4M3"),
        (weight(scale=torch.ones(n, dtype=torch.float64)), "w4a8: scale is float32, N a multiple of 8"),
        (weight(codebook=torch.ones(15)), "w4a8: the codebook is 16 float32 levels"),
        (weight(), "w4a8: the weight's tensors must be on cuda:0"),
    ]
    for w, text in cases:
        with pytest.raises(ValueError, match=text):
            ops._w4a8_weight(w, None, k, torch.bfloat16)


def test_svdq_rank_padding_and_merge():
    assert [svdq_linear.rank(r) for r in (1, 32, 33, 64, 65, 128)] == [32, 32, 64, 64, 128, 128]
    with pytest.raises(ValueError, match="rank 129 exceeds the kernels' 128"):
        svdq_linear.rank(129)
    gen = torch.Generator().manual_seed(0)
    down, up = torch.randn(20, 64, generator=gen), torch.randn(48, 20, generator=gen)
    d, u = svdq_linear.padded(torch, down, up)
    assert d.shape == (32, 64) and u.shape == (48, 32) and d.dtype == u.dtype == torch.bfloat16
    assert d.is_contiguous() and u.is_contiguous()
    assert torch.equal(d[:20], down.to(torch.bfloat16)) and not d[20:].any()
    assert torch.equal(u[:, :20], up.to(torch.bfloat16)) and not u[:, 20:].any()
    roles = {"lowrank_down": d, "lowrank_up": u}
    a, b = torch.randn(8, 64, generator=gen), torch.randn(48, 8, generator=gen)
    m = svdq_linear.merged(torch, roles, a, b)
    assert m["lowrank_down"].shape == (64, 64) and m["lowrank_up"].shape == (48, 64)
    assert torch.equal(m["lowrank_down"][:32], d) and torch.equal(m["lowrank_down"][32:40], a.to(torch.bfloat16))
    assert torch.equal(m["lowrank_up"][:, 32:40], b.to(torch.bfloat16)) and not m["lowrank_up"][:, 40:].any()
    x = torch.randn(5, 64, generator=gen).to(torch.bfloat16).double()
    want = x @ d.double().t() @ u.double().t() + x @ a.to(torch.bfloat16).double().t() @ b.to(torch.bfloat16).double().t()
    got = x @ m["lowrank_down"].double().t() @ m["lowrank_up"].double().t()
    assert torch.allclose(got, want, rtol=0, atol=1e-9)
    assert svdq_linear.merged(torch, roles, torch.zeros(97, 64), torch.zeros(48, 97)) is None


def test_int8_gemv_route_rule():
    """The int8 linear keeps the one-launch GEMV for one row and for short rows, and sends 2-4
    rows with rows x K >= 9216 to quantize + GEMM (the faster route there, same bits)."""
    assert prebuilt.gemv_serves(1, 3072) and prebuilt.gemv_serves(1, 32768)
    assert prebuilt.gemv_serves(2, 3072) and prebuilt.gemv_serves(2, 4096) and prebuilt.gemv_serves(3, 1024)
    assert not prebuilt.gemv_serves(3, 3072) and not prebuilt.gemv_serves(4, 3072)
    assert not prebuilt.gemv_serves(2, 12288) and not prebuilt.gemv_serves(2, 16384)
    assert prebuilt.gemv_serves(2, 4352) and not prebuilt.gemv_serves(2, 4608)
    assert prebuilt.gemv_serves(3, 2816) and not prebuilt.gemv_serves(4, 2304)

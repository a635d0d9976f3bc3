"""The nvfp4 encoded linear on the GPU (`cozyq.nvfp4_linear`, `csrc/nvfp4.hip`).

The W4A16 GEMV (up to 64 rows), the W4A16 GEMM and the decode + library GEMM path
are held to the float64 product of the activations and the exact decoded weight (the oracle's
`decode_nvfp4`, pinned by the reference's nvfp4 vectors), within rtol 2e-2 / atol 1e-2·rms like
every floating output here. Within each kernel a row's bits do not depend on M, and repeat.
"""

from __future__ import annotations

import pytest
import torch

from oracle import laws

pytestmark = pytest.mark.gpu

CUDA = "cuda:0"
RTOL, ATOL = 2e-2, 1e-2


def _weight(n: int, k: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(0, 256, (n, k // 2), generator=g, dtype=torch.int32).to(torch.uint8)
    grid = (torch.rand(n, k // 16, generator=g) * 4 + 0.25).to(torch.float8_e4m3fn)
    second = torch.tensor([0.02])
    exact = laws.decode_nvfp4(codes, grid, second, "row_major", False, False, None, torch.float32)
    blocked = laws.to_blocked(grid.view(torch.uint8)).view(*laws._blocked_shape(n, k // 16))
    return codes, grid, blocked, second, exact


def _close(got: torch.Tensor, want: torch.Tensor) -> None:
    got = got.double().cpu()
    rms = float(want.pow(2).mean().sqrt())
    bad = ((got - want).abs() > ATOL * rms + RTOL * want.abs()).sum()
    assert int(bad) == 0, f"{int(bad)} of {want.numel()} outside tolerance"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k", [(1, 14336, 4096), (2, 14336, 4096), (1, 200, 96), (2, 264, 2080), (1, 12296, 3072),
                                   (3, 200, 1024), (16, 264, 96), (16, 4096, 3072),
                                   (17, 200, 160), (40, 4096, 3072), (64, 1032, 2048), (5, 12288, 640),
                                   (40, 12296, 3072), (64, 14336, 512)])
def test_nvfp4_gemv_against_the_exact_product(dtype, m, n, k):
    from cozyq import prebuilt

    codes, _, blocked, second, exact = _weight(n, k, m + n)
    x = (torch.randn(m, k, generator=torch.Generator().manual_seed(k)) * 0.5).to(dtype)
    ops = prebuilt.library(0)
    got = ops.nvfp4_gemv(x.to(CUDA), codes.to(CUDA), blocked.to(CUDA), second.to(CUDA), dtype)
    torch.cuda.synchronize()
    assert got.shape == (m, n) and got.dtype == dtype
    _close(got, x.double() @ exact.double().t())


@pytest.mark.parametrize("n,sizes", [(4096, (3, 5, 16, 17, 33, 50)), (12288, (5, 9, 16, 17, 33, 50))])
def test_nvfp4_gemv_rows_do_not_depend_on_m(n, sizes):
    """Within a kernel (the streaming form at 1 or 2 rows; the K-split GEMV; the row-block form
    past 4 rows when N gives 192 64-row groups) a row's bits do not depend on M, and repeat."""
    from cozyq import prebuilt

    codes, _, blocked, second, _ = _weight(n, 2048, 9)
    x = torch.randn(64, 2048, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    ops = prebuilt.library(0)
    w, s, g = codes.to(CUDA), blocked.to(CUDA), second.to(CUDA)
    full = ops.nvfp4_gemv(x.to(CUDA), w, s, g, torch.bfloat16).cpu()
    again = ops.nvfp4_gemv(x.to(CUDA), w, s, g, torch.bfloat16).cpu()
    assert torch.equal(full.view(torch.int16), again.view(torch.int16))
    for m in sizes:
        part = ops.nvfp4_gemv(x[:m].to(CUDA), w, s, g, torch.bfloat16).cpu()
        assert torch.equal(part.view(torch.int16), full[:m].view(torch.int16))
    two = ops.nvfp4_gemv(x[:2].to(CUDA), w, s, g, torch.bfloat16).cpu()
    one = ops.nvfp4_gemv(x[:1].to(CUDA), w, s, g, torch.bfloat16).cpu()
    assert torch.equal(one.view(torch.int16), two[:1].view(torch.int16))
    assert torch.equal(two.view(torch.int16), ops.nvfp4_gemv(x[:2].to(CUDA), w, s, g, torch.bfloat16).cpu().view(torch.int16))


@pytest.mark.parametrize("dtype,out_dtype", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                             (torch.bfloat16, torch.float16)])
@pytest.mark.parametrize("m,n,k", [(17, 256, 64), (300, 520, 1024), (256, 1536, 128), (600, 3072, 2048)])
def test_nvfp4_gemm_against_the_exact_product(dtype, out_dtype, m, n, k):
    """The W4A16 GEMM: ragged rows and columns (partial 256x256 tiles), one and two K buffers,
    a bf16 x into an fp16 output."""
    from cozyq import prebuilt

    codes, _, blocked, second, exact = _weight(n, k, m + n)
    x = (torch.randn(m, k, generator=torch.Generator().manual_seed(k)) * 0.5).to(dtype)
    ops = prebuilt.library(0)
    got = ops.nvfp4_gemm(x.to(CUDA), codes.to(CUDA), blocked.to(CUDA), second.to(CUDA), None, out_dtype)
    torch.cuda.synchronize()
    assert got.shape == (m, n) and got.dtype == out_dtype
    _close(got, x.double() @ exact.double().t())


def test_nvfp4_gemm_bias_rows_and_repeats():
    """With a bias; a row's result is bit-identical whatever M is, and repeats bit for bit."""
    from cozyq import prebuilt

    n, k = 776, 512
    codes, _, blocked, second, exact = _weight(n, k, 11)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(520, k, generator=g).to(torch.bfloat16)
    bias = (torch.randn(n, generator=g) * 0.3).to(torch.bfloat16)
    ops = prebuilt.library(0)
    w, s, sc, b = codes.to(CUDA), blocked.to(CUDA), second.to(CUDA), bias.to(CUDA)
    full = ops.nvfp4_gemm(x.to(CUDA), w, s, sc, b, torch.bfloat16).cpu()
    again = ops.nvfp4_gemm(x.to(CUDA), w, s, sc, b, torch.bfloat16).cpu()
    assert torch.equal(full.view(torch.int16), again.view(torch.int16))
    _close(full, x.double() @ exact.double().t() + bias.double())
    for m in (1, 33, 257):
        part = ops.nvfp4_gemm(x[-m:].to(CUDA), w, s, sc, b, torch.bfloat16).cpu()
        assert torch.equal(part.view(torch.int16), full[-m:].view(torch.int16))
    empty = ops.nvfp4_gemm(x[:0].to(CUDA), w, s, sc, b, torch.bfloat16)
    assert empty.shape == (0, n)


@pytest.mark.parametrize("rows", [17, 64, 65, 300])
def test_nvfp4_matmul_gemv_and_gemm_decode_nothing(rows, monkeypatch):
    """Up to 64 rows the GEMV, past them (asked for, K % 64 == 0, N % 8 == 0) the W4A16 GEMM: no
    decoded transient either way."""
    from cozyq import nvfp4_linear, prebuilt

    n, k = 264, 192
    codes, _, blocked, second, exact = _weight(n, k, 6)
    ops = prebuilt.library(0)
    monkeypatch.setattr(type(ops), "decode_table", lambda *a, **kw: pytest.fail("decoded the weight"))
    x = torch.randn(rows, k, generator=torch.Generator().manual_seed(8)).to(torch.float16)
    got = nvfp4_linear.matmul(torch, x.to(CUDA), codes.to(CUDA), blocked.to(CUDA), None,
                              second.to(CUDA), torch.float32, gemm=True)  # fmt: skip
    torch.cuda.synchronize()
    assert got.shape == (rows, n) and got.dtype == torch.float32
    _close(got, x.double() @ exact.double().t())


@pytest.mark.parametrize("rows", [65, 100])
def test_nvfp4_matmul_more_rows_decodes_per_chunk(rows, monkeypatch):
    """Past 64 rows by default: the weight decoded per 128-row chunk (here forced small, so the
    last chunk is partial) and the library GEMM."""
    from cozyq import nvfp4_linear

    n, k = 300, 1024
    codes, grid, blocked, second, exact = _weight(n, k, 3)
    monkeypatch.setattr(nvfp4_linear, "_DECODE_CHUNK", 2 * k * 128)
    x = torch.randn(2, rows, k, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    got = nvfp4_linear.matmul(torch, x.to(CUDA), codes.to(CUDA), blocked.to(CUDA), None,
                              second.to(CUDA), torch.float32)  # fmt: skip
    torch.cuda.synchronize()
    assert got.shape == (2, rows, n) and got.dtype == torch.float32
    want = x.double().reshape(-1, k) @ exact.double().t()
    _close(got.reshape(-1, n), want)


@pytest.mark.parametrize("layout,order,mode", [("row_major", "low_first", "multiply"),
                                               ("cublas_128x4", "high_first", "divide")])
@pytest.mark.parametrize("rows", [1, 40])
def test_nvfp4_leaf_forward(layout, order, mode, rows):
    """The provider's leaf from stored parts of either convention, with a bias."""
    from cozyq import leaves

    n, k = 256, 512
    g = torch.Generator().manual_seed(5)
    codes = torch.randint(0, 256, (n, k // 2), generator=g, dtype=torch.int32).to(torch.uint8)
    grid = (torch.rand(n, k // 16, generator=g) * 4 + 0.25).to(torch.float8_e4m3fn)
    second = torch.tensor(0.05 if mode == "multiply" else 20.0)
    exact = laws.decode_nvfp4(codes, grid, second, "row_major", order == "high_first",
                              mode == "divide", None, torch.float32)  # fmt: skip
    scale = grid if layout == "row_major" else laws.to_blocked(grid.view(torch.uint8)).view(
        *laws._blocked_shape(n, k // 16)).view(torch.float8_e4m3fn)  # fmt: skip
    params = (("block_size", 16), ("global_scale", mode), ("nibble_order", order),
              ("scale_layout", layout))  # fmt: skip
    lin = torch.nn.Linear(k, n, bias=True)
    lin.bias.data = (torch.randn(n, generator=g) * 0.1)
    lin = lin.to(CUDA).to(torch.bfloat16)
    leaf = leaves.Nvfp4NativeLeaf("nvfp4", params).leaf(
        torch, {"weight": codes.to(CUDA), "scale": scale.to(CUDA), "scale_2": second.to(CUDA)},
        lin, torch.bfloat16)  # fmt: skip
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16)
    got = leaf(x.to(CUDA))
    torch.cuda.synchronize()
    want = x.double() @ exact.double().t() + lin.bias.detach().double().cpu()
    _close(got, want)

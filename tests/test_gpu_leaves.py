"""The encoded leaves end to end on the GPU (`cozyq.leaves`): each provider's leaf against the
CPU oracle, and the reference's call-graph behaviours — shared operands (`quantize_once`),
producer operands (`int8_rows`), writing into a sibling group's column range (`out=`), the
decode-row path and autocast. int8 outputs bit-exact; the others within ATOL·rms + RTOL·|x|."""

from __future__ import annotations

import pytest
import torch

from cozyq import int8_linear, leaves, operands
from oracle import laws

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-2, 2e-2
DEV = "cuda:0"


class _Linear(torch.nn.Module):
    def __init__(self, bias: torch.Tensor | None) -> None:
        super().__init__()
        self.bias = bias


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def activations(m: int, k: int, seed: int, dtype=torch.bfloat16) -> torch.Tensor:
    gen = _gen(seed)
    x = torch.randn(m, k, generator=gen)
    x[:, torch.randperm(k, generator=gen)[: max(1, k // 100)]] *= 20
    return x.to(dtype)


def assert_close(got: torch.Tensor, exact: torch.Tensor) -> None:
    got, exact = got.double().cpu(), exact.double().cpu()
    rms = exact.pow(2).mean().sqrt().item()
    worst = ((got - exact).abs() - (ATOL * rms + RTOL * exact.abs())).max().item()
    assert worst <= 0, f"max excess {worst:.3g} (rms {rms:.3g})"


def int8_leaf(n: int, k: int, seed: int, bias: bool = True):
    data, scale = laws.int8_weight_rotated(torch.randn(n, k, generator=_gen(seed)) * 0.02, 256)
    b = (torch.randn(n, generator=_gen(seed + 1)) * 0.1).to(torch.bfloat16) if bias else None
    leaf = leaves.Int8ConvRotNativeLeaf().leaf(
        torch, {"weight": data.to(DEV), "scale": scale.to(DEV)},
        _Linear(None if b is None else b.to(DEV)), torch.bfloat16)  # fmt: skip
    return leaf, data, scale, b


@pytest.mark.parametrize("m", [3, 300])
def test_int8_leaf_bit_exact(m):
    leaf, data, scale, b = int8_leaf(520, 1024, 71)
    x = activations(m, 1024, 72 + m)
    got = leaf(x.to(DEV))
    assert got.dtype == torch.bfloat16 and got.shape == (m, 520)
    assert torch.equal(got.cpu(), laws.int8_linear(x, data, scale, b, torch.bfloat16, rotation=256))


def test_int8_leaves_share_one_quantization(monkeypatch):
    """q, k and v of one input quantize it once inside `quantize_once`, and each output is what
    the leaf computes alone."""
    x = activations(200, 512, 81).to(DEV)
    trio = [int8_leaf(256, 512, 82 + 7 * i)[0] for i in range(3)]
    alone = [leaf(x) for leaf in trio]
    lib = int8_linear.library(0)
    calls = []
    original = type(lib).int8_quantize

    def counting(self, *args, **kwargs):
        calls.append(1)
        return original(self, *args, **kwargs)

    monkeypatch.setattr(type(lib), "int8_quantize", counting)
    with operands.quantize_once(x):
        shared = [leaf(x) for leaf in trio]
    assert len(calls) == 1
    for a, s in zip(alone, shared):
        assert torch.equal(a, s)


def test_int8_rows_operand_and_out_into_a_column_range():
    leaf, data, scale, b = int8_leaf(264, 768, 91)
    x = activations(130, 768, 92)
    xd = x.to(DEV)
    pre = operands.int8_rows(xd, (leaf,))
    assert isinstance(pre, operands.PreQuantized) and pre.provider == operands.INT8_CONVROT
    want = laws.int8_linear(x, data, scale, b, torch.bfloat16, rotation=256)
    assert torch.equal(leaf(xd, prequantized=pre).cpu(), want)
    packed = torch.zeros(130, 3 * 264, dtype=torch.bfloat16, device=DEV)
    got = leaf(xd, out=packed[:, 264:528])
    assert got.data_ptr() == packed[:, 264:528].data_ptr()
    assert torch.equal(packed[:, 264:528].cpu(), want)
    assert packed[:, :264].eq(0).all() and packed[:, 528:].eq(0).all()
    assert leaf(xd, prequantized=pre, out=packed[:, :264]).data_ptr() == packed.data_ptr()


def test_int8_rows_with_a_prologue():
    """`int8_rows` with the producer prologue (RMS norm, a two-row modulation table, tanh-GELU)
    hands the leaf rows quantized in one pass; the linear matches the law on the prologue's
    rows within tolerance (the prologue's transcendentals are the platform's)."""
    leaf, data, scale, b = int8_leaf(264, 768, 93)
    x = activations(130, 768, 94)
    mod = (torch.randn(2, 768, generator=_gen(95)) * 0.2).to(torch.bfloat16)
    pre = operands.int8_rows(x.to(DEV), (leaf,), norm="rms", eps=1e-6, scale=mod.to(DEV),
                             activation="gelu_tanh")  # fmt: skip
    assert isinstance(pre, operands.PreQuantized) and pre.shape == (130, 768)
    got = leaf(x.to(DEV), prequantized=pre)
    rows = laws.prologue(x, scale=mod, norm=laws.NORM_RMS, eps=1e-6,
                         activation=laws.ACT_GELU_TANH)  # fmt: skip
    assert_close(got, laws.int8_exact(rows, data, scale, b, 256))
    gated = activations(130, 2 * 768, 96)
    pre = operands.int8_rows(gated.to(DEV), (leaf,), activation="situ")
    assert isinstance(pre, operands.PreQuantized) and pre.shape == (130, 768)
    got = leaf(gated[:, :768].to(DEV), prequantized=pre)
    assert_close(got, laws.int8_exact(laws.prologue(gated, activation=laws.ACT_SITU), data,
                                      scale, b, 256))  # fmt: skip


def test_w4a8_leaf_shares_the_int8_operand(monkeypatch):
    """The w4a8 leaf (`W4a8NativeLeaf`) takes int8.convrot's operand: its forward equals the int8
    law on the unpacked levels, bit for bit, and an int8 leaf beside it reads the same shared
    operand."""
    from cozyq import prebuilt

    n, k = 264, 1024
    gen = _gen(97)
    codes = torch.randint(0, 256, (n, k // 2), generator=gen, dtype=torch.uint8)
    gs = (torch.randn(n, k // 16, generator=gen).abs() * 40 + 16).clamp(max=440).to(torch.float8_e4m3fn)
    scale = (torch.randn(n, generator=gen).abs() + 0.5) * 1e-3
    book = torch.tensor(laws.W4A8_CODEBOOK)
    b = (torch.randn(n, generator=gen) * 0.1).to(torch.bfloat16)
    provider = leaves.W4a8NativeLeaf()
    assert provider.supports((n, k), {"group_size": 16, "rotation": "kron_regular_h4",
                                      "rotation_size": 256}) == ""  # fmt: skip
    leaf = provider.leaf(torch, {"weight": codes.to(DEV), "group_scale": gs.to(DEV),
                                 "scale": scale.to(DEV), "codebook": book.to(DEV)},
                         _Linear(b.to(DEV)), torch.bfloat16)  # fmt: skip
    assert leaf.operand == operands.INT8_CONVROT
    levels = laws.w4a8_unpack(codes, gs, book)
    for m in (3, 130):
        x = activations(m, k, 98 + m)
        want = laws.int8_linear(x, levels, scale, b, torch.bfloat16, rotation=256)
        assert torch.equal(leaf(x.to(DEV)).cpu(), want)
    int8, _, _, _ = int8_leaf(264, k, 99)
    x = activations(130, k, 100).to(DEV)
    alone = (leaf(x), int8(x))
    lib = int8_linear.library(0)
    calls = []
    original = type(lib).int8_quantize

    def counting(self, *args, **kwargs):
        calls.append(1)
        return original(self, *args, **kwargs)

    monkeypatch.setattr(type(lib), "int8_quantize", counting)
    with operands.quantize_once(x):
        shared = (leaf(x), int8(x))
    assert len(calls) == 1
    assert all(torch.equal(a, s) for a, s in zip(alone, shared))
    assert leaf.roles()["group_scale"].dtype == torch.float8_e4m3fn and leaf.codebook is not None


def test_int8_leaf_autocast_dtype():
    leaf, data, scale, _ = int8_leaf(256, 512, 95, bias=False)
    x = activations(40, 512, 96)
    with torch.autocast("cuda", dtype=torch.float16):
        got = leaf(x.to(DEV))
    assert got.dtype == torch.float16
    want = laws.int8_linear(x.to(torch.float16), data, scale, None, torch.float16, rotation=256)
    assert torch.equal(got.cpu(), want)


@pytest.mark.parametrize("m", [1, 16, 300])
def test_fp8_leaf_within_tolerance(m):
    n, k = 1032, 2048
    data, scale = laws.fp8_weight(torch.randn(n, k, generator=_gen(101)) * 0.02)
    b = (torch.randn(n, generator=_gen(102)) * 0.1).to(torch.bfloat16)
    leaf = leaves.RowwiseNativeLeaf().leaf(torch, {"weight": data.to(DEV), "scale": scale.to(DEV)},
                                           _Linear(b.to(DEV)), torch.bfloat16)  # fmt: skip
    x = activations(m, k, 103 + m)
    got = leaf(x.to(DEV))
    assert got.shape == (m, n) and leaf.operand == operands.ROWWISE_FP8
    assert_close(got, laws.fp8_exact(x, data, scale, b))


def test_mx_leaf_within_tolerance():
    n, k, m = 264, 1024, 300
    data, wbyte = laws.mx_quantize(torch.randn(n, k, generator=_gen(111)) * 0.02)
    b = (torch.randn(n, generator=_gen(112)) * 0.1).to(torch.bfloat16)
    provider = leaves.MicroScaledNativeLeaf(params=(("scale_layout", "cublas_128x4"),))
    leaf = provider.leaf(torch, {"weight": data.to(DEV), "scale": laws.to_blocked(wbyte).to(DEV)},
                         _Linear(b.to(DEV)), torch.bfloat16)  # fmt: skip
    x = activations(m, k, 113)
    assert_close(leaf(x.to(DEV)), laws.mx_exact(x, data, wbyte, b))


def test_svdq_leaf_within_tolerance():
    n, k, r, m = 520, 1024, 32, 260
    gen = _gen(121)
    p = torch.rand(k, generator=gen) * 1.5 + 0.5
    down = (torch.randn(r, k, generator=gen) * 0.02).to(torch.bfloat16)
    up = (torch.randn(n, r, generator=gen) * 0.02).to(torch.bfloat16)
    codes, scales = laws.svdq_weight(torch.randn(n, k, generator=gen) * 0.02, p, down, up)
    b = (torch.randn(n, generator=gen) * 0.1).to(torch.bfloat16)
    parts = {"weight": codes, "scale": scales, "pre_quant_scale": p, "lowrank_down": down,
             "lowrank_up": up}  # fmt: skip
    leaf = leaves.SvdqInt4NativeLeaf().leaf(torch, {key: v.to(DEV) for key, v in parts.items()},
                                            _Linear(b.to(DEV)), torch.bfloat16)  # fmt: skip
    x = activations(m, k, 122)
    assert_close(leaf(x.to(DEV)), laws.svdq_exact(x, p, codes, scales, down, up, b))

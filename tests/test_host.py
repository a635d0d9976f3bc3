"""The host layer on the CPU (no kernels run): the leaf providers' surface, leaf construction
and buffers, operand sharing (`quantize_once`, `shared_operand`, `int8_rows`), the 128x4 scale
layout against the oracle's, and that a leaf refuses to compute off the GPU instead of falling
back."""

from __future__ import annotations

import pytest
import torch

from cozyq import layout, leaves, operands
from oracle import laws


class _Linear(torch.nn.Module):
    def __init__(self, n: int, k: int, bias: bool) -> None:
        super().__init__()
        self.weight = torch.nn.Parameter(torch.zeros(n, k))
        self.bias = torch.nn.Parameter(torch.ones(n)) if bias else None


def test_providers_surface_and_launch_table():
    table = leaves.launch_providers()
    assert set(table) == {"fp8.rowwise", "int8.convrot", "w4a8.convrot", "svdq.nvfp4",
                          "svdq.int4g64", "mxfp8", "nvfp4"}  # fmt: skip
    names = {p.name for ps in table.values() for p in ps}
    assert names == {operands.ROWWISE_FP8, operands.INT8_CONVROT, leaves.W4A8, leaves.MXFP8,
                     leaves.SVDQ, leaves.SVDQ_INT4, leaves.NVFP4}  # fmt: skip
    assert leaves.SVDQ == "cozy.svdq-nvfp4.native-leaf/1"  # internal/encoding/leaves.py:72
    assert leaves.OPERANDS[leaves.W4A8] == operands.INT8_CONVROT
    for scheme, (provider,) in table.items():
        assert provider.encoding == scheme
        assert provider.route == "encoded_gemm"
        assert provider.device_predicate == "rocm.gfx950"
        assert provider.output_dtype_rule == "contract"
        assert {"weight", "scale"} <= provider.required
        assert leaves.serves(provider, "gfx950") and not leaves.serves(provider, "gfx942")
        with pytest.raises(AssertionError):
            provider.decode(torch, {}, torch.empty(0))


def test_svdq_nvfp4_leaf_surface_and_supports():
    """`internal/encoding/leaves.py:1267-1330`: roles, out dtypes, nvfp4's block law, and this
    GEMM's K % 64 and N % 8; the rank helpers of `internal/svdq_linear.py:266-299`."""
    from cozyq import svdq_linear

    sv = leaves.SvdqNvfp4NativeLeaf()
    assert sv.encoding == "svdq.nvfp4" and sv.suite == "svdq-nvfp4-native"
    assert sv.required == {"weight", "scale", "scale_2", "pre_quant_scale", "lowrank_down", "lowrank_up"}
    assert sv.optional == {"input_scale", "channel_scale"}
    assert sv.out_dtypes == {"bfloat16", "float16"}
    ok = {"block_size": 16, "global_scale": "multiply", "nibble_order": "low_first",
          "scale_layout": "row_major"}  # fmt: skip
    assert sv.supports([3072, 3072], ok) == ""
    assert "K % 64" in sv.supports([3072, 3040], ok)
    assert "N % 8" in sv.supports([3074, 3072], ok)
    assert sv.supports([2, 3072, 3072], ok)
    assert sv.supports([3072, 3072], {**ok, "block_size": 32})
    assert [svdq_linear.rank(r) for r in (1, 32, 33, 64, 65, 128)] == [32, 32, 64, 64, 128, 128]
    with pytest.raises(ValueError):
        svdq_linear.rank(129)
    down, up = torch.ones(4, 64), torch.ones(8, 4)
    d, u = svdq_linear.padded(torch, down, up)
    assert d.shape == (32, 64) and u.shape == (8, 32) and d.dtype == u.dtype == torch.bfloat16
    assert not d[4:].any() and not u[:, 4:].any()
    roles = {"lowrank_down": d, "lowrank_up": u}
    m = svdq_linear.merged(torch, roles, torch.full((16, 64), 2.0), torch.full((8, 16), 3.0))
    assert m is not None and m["lowrank_down"].shape == (64, 64) and m["lowrank_up"].shape == (8, 64)
    assert svdq_linear.merged(torch, roles, torch.ones(100, 64), torch.ones(8, 100)) is None


def test_nvfp4_leaf_surface_and_supports():
    """`internal/encoding/leaves.py:1069-1134`: roles, out dtypes, the decode's block law, K % 32
    and N % 8."""
    nv = leaves.Nvfp4NativeLeaf()
    ok = {"block_size": 16, "global_scale": "multiply", "nibble_order": "low_first",
          "scale_layout": "row_major"}  # fmt: skip
    assert nv.name == "cozy.nvfp4.native-leaf/1" and nv.suite == "nvfp4-native"
    assert nv.required == {"weight", "scale", "scale_2"} and nv.optional == {"input_scale"}
    assert nv.supports((64, 256), ok) == ""
    assert "K % 32" in nv.supports((64, 48), ok)
    assert "N % 8" in nv.supports((60, 256), ok)
    assert "expected one of" in nv.supports((64, 256), {**ok, "global_scale": "add"})
    assert "rank-2" in nv.supports((2, 64, 256), ok)


def test_nvfp4_leaf_holds_the_kernels_layout():
    """Fill: a high-first weight is held low first, row-major scales in 128x4 tiles, a divide
    second level as its reciprocal (`internal/encoding/leaves.py:1172-1203`)."""
    torch.manual_seed(0)
    codes = torch.randint(0, 256, (8, 32), dtype=torch.uint8)
    grid = torch.randint(1, 120, (8, 4), dtype=torch.uint8)
    nv = leaves.Nvfp4NativeLeaf("nvfp4", (("block_size", 16), ("global_scale", "divide"),
                                          ("nibble_order", "high_first"),
                                          ("scale_layout", "row_major")))  # fmt: skip
    leaf = nv.leaf(torch, {"weight": codes, "scale": grid.view(torch.float8_e4m3fn),
                           "scale_2": torch.tensor(4.0)}, _Linear(8, 64, False), torch.bfloat16)  # fmt: skip
    assert torch.equal(leaf.weight, (codes << 4) | (codes >> 4))
    assert torch.equal(leaf.weight_scale.view(torch.uint8).reshape(-1), laws.to_blocked(grid))
    assert float(leaf.weight_scale_2) == 0.25
    assert (leaf.in_features, leaf.out_features) == (64, 8)
    with pytest.raises(ValueError, match="on the GPU"):
        leaf(torch.zeros(2, 64, dtype=torch.bfloat16))


def test_w4a8_supports_messages():
    """`internal/encoding/leaves.py:1004-1013`: group 16, the 256 rotation, K % 256, N % 8."""
    w4 = leaves.W4a8NativeLeaf()
    ok = {"group_size": 16, "rotation": "kron_regular_h4", "rotation_size": 256}
    assert w4.supports((64, 512), ok) == ""
    assert "reads" in w4.supports((64, 512), {**ok, "group_size": 32})
    assert "K % 256" in w4.supports((64, 640), ok)
    assert "N % 8" in w4.supports((60, 512), ok)
    assert w4.optional == frozenset({"codebook"})


def test_supports_messages():
    fp8 = leaves.RowwiseNativeLeaf()
    assert fp8.supports((64, 128), {}) == ""
    assert "K divisible by 16" in fp8.supports((64, 120), {})
    assert "rank-2" in fp8.supports((4, 4, 4), {})
    i8 = leaves.Int8ConvRotNativeLeaf()
    assert i8.supports((64, 512), {"rotation_size": 256}) == ""
    assert "256-groups" in i8.supports((64, 512), {"rotation_size": 128})
    assert "divisible by 8" in i8.supports((60, 512), {"rotation_size": 256})
    mx = leaves.MicroScaledNativeLeaf()
    assert mx.supports((64, 256), {}) == "" and "128-element" in mx.supports((64, 96), {})
    sv = leaves.SvdqInt4NativeLeaf()
    assert sv.supports((64, 96), {"rank": 32}) == ""
    assert "ranks" in sv.supports((64, 96), {"rank": 8})
    assert "K % 64" in sv.supports((64, 40), {})


def test_native_leaf_buffers_roles_and_refusal_off_gpu():
    provider = leaves.Int8ConvRotNativeLeaf()
    data = torch.randint(-127, 128, (16, 256), dtype=torch.int8)
    scale = torch.rand(16, dtype=torch.float64)
    leaf = provider.leaf(torch, {"weight": data, "scale": scale}, _Linear(16, 256, True), torch.bfloat16)
    assert isinstance(leaf, torch.nn.Module)
    assert leaf.data is data and leaf.scale.dtype == torch.float32  # the kernels read f32
    assert not hasattr(leaf, "weight")  # no `.weight`: BUFFERS maps it to `data`
    assert set(leaf.roles()) == {"weight", "scale"}
    assert leaf.in_features == 256 and leaf.out_features == 16
    assert leaf.operand == operands.INT8_CONVROT and leaf.WRITES_INTO
    assert "provider='cozy.int8-convrot256.native-leaf/1'" in repr(leaf)
    assert leaf.bias is not None and "_logical_dtype" not in leaf.state_dict()
    x = torch.randn(8, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="gfx950"):
        leaf(x)  # no CPU fallback: the kernels are the only implementation


def test_fp8_and_svdq_leaves_refuse_off_gpu():
    fp8 = leaves.RowwiseNativeLeaf().leaf(
        torch, {"weight": torch.zeros(8, 64, dtype=torch.float8_e4m3fn), "scale": torch.ones(8)},
        _Linear(8, 64, False), torch.bfloat16)  # fmt: skip
    with pytest.raises(ValueError, match="gfx950"):
        fp8(torch.randn(2, 64, dtype=torch.bfloat16))
    parts = {"weight": torch.zeros(8, 32, dtype=torch.uint8), "scale": torch.ones(8, 1),
             "pre_quant_scale": torch.ones(64), "lowrank_down": torch.zeros(16, 64),
             "lowrank_up": torch.zeros(8, 16)}  # fmt: skip
    sv = leaves.SvdqInt4NativeLeaf().leaf(torch, parts, _Linear(8, 64, False), torch.bfloat16)
    assert sv.in_features == 64 and sv.scale.dtype == torch.float16
    with pytest.raises(ValueError, match="gfx950"):
        sv(torch.randn(2, 64, dtype=torch.bfloat16))


def test_mx_leaf_untiles_cublas_scales():
    gen = torch.Generator().manual_seed(3)
    n, k = 136, 256
    grid = torch.randint(0, 255, (n, k // 32), generator=gen, dtype=torch.uint8)
    weight = torch.zeros(n, k, dtype=torch.float8_e4m3fn)
    tiled = laws.to_blocked(grid)
    provider = leaves.MicroScaledNativeLeaf(params=(("scale_layout", "cublas_128x4"),))
    leaf = provider.leaf(torch, {"weight": weight, "scale": tiled}, _Linear(n, k, False), torch.bfloat16)
    assert torch.equal(leaf.scale, grid)
    plain = leaves.MicroScaledNativeLeaf().leaf(torch, {"weight": weight, "scale": grid},
                                                _Linear(n, k, False), torch.bfloat16)  # fmt: skip
    assert torch.equal(plain.scale, grid)


@pytest.mark.parametrize("rows,cols", [(1, 1), (128, 4), (130, 7), (300, 96), (17, 384)])
def test_layout_matches_oracle(rows, cols):
    grid = torch.randint(0, 256, (rows, cols), dtype=torch.uint8)
    assert torch.equal(layout.to_blocked(torch, grid), laws.to_blocked(grid))
    assert torch.equal(layout.from_blocked(torch, laws.to_blocked(grid), rows, cols), grid)
    with pytest.raises(ValueError):
        layout.from_blocked(torch, grid.reshape(-1)[:-1], rows, cols) if rows * cols > 1 else \
            layout.from_blocked(torch, torch.zeros(3, dtype=torch.uint8), rows, cols)


def _op(counter: list[int], x: torch.Tensor, provider: str):
    def make():
        counter.append(1)
        return operands.PreQuantized(x, torch.ones(1), tuple(x.shape), provider)

    return make


def test_quantize_once_scope_shares_per_provider():
    x, y = torch.randn(4, 8), torch.randn(4, 8)
    made: list[int] = []
    with operands.quantize_once(x, None):
        a = operands.shared_operand(x, operands.INT8_CONVROT, _op(made, x, operands.INT8_CONVROT))
        b = operands.shared_operand(x, operands.INT8_CONVROT, _op(made, x, operands.INT8_CONVROT))
        c = operands.shared_operand(x, operands.ROWWISE_FP8, _op(made, x, operands.ROWWISE_FP8))
        assert operands.shared_operand(y, operands.INT8_CONVROT, _op(made, y, "p")) is None  # no consumer
    assert a is b and c is not a and len(made) == 2  # one per provider; y (no consumer) none


def test_siblings_share_then_learn_their_group():
    class Leaf:
        pass

    q, k, v = Leaf(), Leaf(), Leaf()
    x = torch.randn(4, 8)
    made: list[int] = []
    p = operands.INT8_CONVROT
    first = [operands.shared_operand(x, p, _op(made, x, p), leaf) for leaf in (q, k, v)]
    assert first[0] is first[1] is first[2] and len(made) == 1
    x2 = torch.randn(4, 8)  # a new input retires the held operand; q learns its group of 3
    operands.shared_operand(x2, p, _op(made, x2, p), q)
    assert operands.group_size(q) == 3 and len(made) == 2
    x.add_(1)  # an in-place change is never served stale
    operands.shared_operand(x, p, _op(made, x, p), q)
    assert len(made) == 3


def test_int8_rows_declines_foreign_consumers():
    x = torch.randn(4, 256, dtype=torch.bfloat16)
    assert operands.int8_rows(x, ()) is None
    assert operands.int8_rows(x, (torch.nn.Linear(256, 8),)) is None
    leaf = leaves.Int8ConvRotNativeLeaf().leaf(
        torch, {"weight": torch.zeros(8, 256, dtype=torch.int8), "scale": torch.ones(8)},
        _Linear(8, 256, False), torch.bfloat16)  # fmt: skip
    assert operands.int8_rows(x, (leaf,)) is None  # a CPU tensor: the caller runs its own ops
    with pytest.raises(ValueError, match="gate"):
        operands.int8_rows(x, (leaf,), activation="situ", norm="rms")


def test_sharing_groups_grow_exhaust_and_hold_nothing_alone():
    """Rules S2–S5 in sequence: a learned group of 3 holds its operand for exactly two more
    reads; one more reader of the same unchanged input grows the maker's group to 4; a maker
    learned to read alone holds nothing; a freed input drops its operand and its maker learns;
    inference tensors and consumer-less asks share nothing."""
    import gc

    class Leaf:
        pass

    p = operands.INT8_CONVROT
    q, k, v, w = Leaf(), Leaf(), Leaf(), Leaf()
    made: list[int] = []
    x = torch.randn(4, 8)
    for leaf in (q, k, v):
        operands.shared_operand(x, p, _op(made, x, p), leaf)
    x2 = torch.randn(4, 8)
    operands.shared_operand(x2, p, _op(made, x2, p), w)  # drops q's operand: q's group is 3
    assert operands.group_size(q) == 3 and len(made) == 2
    x3 = torch.randn(4, 8)
    got = [operands.shared_operand(x3, p, _op(made, x3, p), leaf) for leaf in (q, k, v)]
    assert got[0] is got[1] is got[2] and len(made) == 3  # w's operand dropped: w read alone
    assert operands.group_size(w) == 1
    again = operands.shared_operand(x3, p, _op(made, x3, p), w)  # a fourth reader after the group
    assert again is not got[0] and len(made) == 4 and operands.group_size(q) == 4
    x4 = torch.randn(4, 8)
    operands.shared_operand(x4, p, _op(made, x4, p), w)  # w reads alone: nothing held
    assert operands.shared_operand(x4, p, _op(made, x4, p), k) is not None and len(made) == 6
    x5 = torch.randn(4, 8)
    payload = torch.zeros(4, 8)  # an operand that does not keep x5 alive
    operands.shared_operand(x5, p, _op(made, payload, p), v)  # v's group unknown: held
    del x5
    gc.collect()
    assert operands.group_size(v) == 1  # dropped with its input; v learned it read alone
    with torch.inference_mode():
        xi = torch.randn(4, 8)
    assert operands.shared_operand(xi, p, _op(made, xi, p), q) is None
    assert operands.shared_operand(x4, p, _op(made, x4, p), None) is None
    assert len(made) == 7

"""The allocation-free fused linear (`cozyq_linear_noalloc`: its counters in the library's own
device array) against the workspace entry point (`cozyq_linear`), through the C ABI: bit for bit,
on two calls in a row, the second with fewer rows, and a size past the array refused."""

from __future__ import annotations

import pytest
import torch

from oracle import laws

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _operands(m: int, n: int, k: int, seed: int):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=gen)
    x[:, torch.randperm(k, generator=gen)[: k // 100]] *= 20
    w = torch.randn(n, k, generator=gen) * 0.02
    data, scale = laws.int8_weight_rotated(w, 128)
    bias = (torch.randn(n, generator=gen) * 0.1).to(torch.bfloat16)
    return x.to(torch.bfloat16).to(DEV), data.to(DEV), scale.to(DEV), bias.to(DEV)


def _call(lib, fn, x, data, scale, bias, work):
    m, k = x.shape
    n = data.shape[0]
    q = torch.empty(m, k, dtype=torch.int8, device=DEV)
    s = torch.empty(m, dtype=torch.float32, device=DEV)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    args = [0, x.data_ptr(), 0, 128, q.data_ptr(), s.data_ptr(), data.data_ptr(), scale.data_ptr(),
            bias.data_ptr(), out.data_ptr(), n, 0, m, n, k, 1]
    if work is not None:
        args.append(work.data_ptr())
    code = fn(*args, torch.cuda.current_stream().cuda_stream)
    assert code == 0, code
    return out, q, s


def test_linear_noalloc_matches_the_workspace_entry_point():
    from cozyq import _lib

    lib = _lib.load()
    for m, n, k, seed in ((2309, 1032, 3072, 1), (300, 520, 1024, 2)):  # the second call smaller
        x, data, scale, bias = _operands(m, n, k, seed)
        work = torch.zeros(int(lib.cozyq_linear_workspace_bytes(m)) // 4, dtype=torch.int32, device=DEV)
        want = _call(lib, lib.cozyq_linear, x, data, scale, bias, work)
        got = _call(lib, lib.cozyq_linear_noalloc, x, data, scale, bias, None)
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b)
    rows = lib.cozyq_linear_noalloc_max_rows()
    assert rows == 262144
    x, data, scale, bias = _operands(16, 264, 256, 3)
    args = [0, x.data_ptr(), 0, 128, x.data_ptr(), scale.data_ptr(), data.data_ptr(), scale.data_ptr(),
            bias.data_ptr(), x.data_ptr(), 264, 0, rows + 1, 264, 256, 0, torch.cuda.current_stream().cuda_stream]
    refused = lib.cozyq_linear_noalloc(*args)  # refused before anything runs
    assert _lib.error_name(refused) == "hipErrorInvalidValue"


def test_linear_noalloc_reports_a_wait_that_gives_up():
    """The failure path of the fused kernel's bounded wait through the allocation-free entry
    point, forced from the host (every workgroup gives up before it waits, so every kernel exits
    normally): NaN outputs, the status read reports it (hipErrorLaunchTimeOut) once; the next
    call, at the default limit, equals the workspace entry point and reads back clean."""
    from cozyq import _lib

    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    x, data, scale, bias = _operands(700, 520, 1024, 4)
    lib.cozyq_linear_test_spin_limit(-1)
    try:
        out, _, _ = _call(lib, lib.cozyq_linear_noalloc, x, data, scale, bias, None)
        torch.cuda.synchronize()
    finally:
        lib.cozyq_linear_test_spin_limit(0)
    assert torch.isnan(out.float()).all()
    assert _lib.error_name(lib.cozyq_linear_noalloc_status(0, stream)) == "hipErrorLaunchTimeOut"
    assert lib.cozyq_linear_noalloc_status(0, stream) == 0
    got = _call(lib, lib.cozyq_linear_noalloc, x, data, scale, bias, None)
    work = torch.zeros(int(lib.cozyq_linear_workspace_bytes(700)) // 4, dtype=torch.int32, device=DEV)
    want = _call(lib, lib.cozyq_linear, x, data, scale, bias, work)
    torch.cuda.synchronize()
    assert lib.cozyq_linear_noalloc_status(0, stream) == 0
    for a, b in zip(got, want):
        assert torch.equal(a, b)

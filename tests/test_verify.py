"""The card's self-check (`cozyq.verify`) on the CPU: its float64 laws against the oracle's, its
verdict arithmetic, and its crash markers (a probe that ends its process is refused by the next
one). The probes themselves run on the GPU (`test_gpu_verify.py`)."""

from __future__ import annotations

import math

import pytest
import torch

from cozyq import verify
from oracle import laws


def test_rotation_is_the_formats_hadamard():
    """The probe's 256-point rotation matrix against the oracle's staged transform
    (`internal/encoding/formats.py:657-671`): x·R·16 equals the unnormalized H256 sums."""
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(7, 512, generator=gen, dtype=torch.float64)
    r = verify.rotation(torch, "cpu")
    got = (x.reshape(7, 2, 256) @ r).reshape(7, 512) * 16.0
    assert torch.allclose(got, laws.hadamard(x, 256), rtol=0, atol=1e-12)
    assert torch.allclose(r @ r.t(), torch.eye(256, dtype=torch.float64), atol=1e-14)


def test_laws_match_the_oracle():
    """int8_law within float32-rotation noise of the oracle's exact int8 product (codes may move
    at rounding ties), fp8_law the oracle's exact fp8 product bit for bit."""
    gen = torch.Generator().manual_seed(6)
    x = torch.randn(9, 512, generator=gen).to(torch.bfloat16)
    data = torch.randint(-127, 128, (40, 512), generator=gen, dtype=torch.int8)
    scale = torch.rand(40, generator=gen) * 1e-3 + 5e-4
    bias = torch.randn(40, generator=gen).to(torch.bfloat16)
    want = laws.int8_exact(x, data, scale, bias)
    got = verify.int8_law(torch, x, data, scale, bias)
    assert verify.error(torch, got, want) < 1e-3
    f8, f8s = laws.fp8_weight(torch.randn(40, 512, generator=gen) * 0.02)
    assert torch.equal(verify.fp8_law(torch, x, f8, f8s, bias), laws.fp8_exact(x, f8, f8s, bias))


def test_error_and_budget():
    want = torch.tensor([3.0, 4.0], dtype=torch.float64)
    assert verify.error(torch, want, want) == 0.0
    assert verify.error(torch, torch.tensor([3.0, 4.05], dtype=torch.float64), want) == pytest.approx(1e-2)
    assert verify.error(torch, torch.tensor([math.nan, 4.0]), want) == math.inf
    ok = verify.within({"a": 1e-3, "b": 9e-3})
    assert ok.ok and "9.00e-03 at b" in ok.detail
    bad = verify.within({"a": 1e-3, "b": 2e-2})
    assert not bad.ok and "at b" in bad.detail
    assert not verify.within({}).ok
    assert not verify.within({"nan": math.inf}).ok


@pytest.fixture()
def markers(tmp_path, monkeypatch):
    monkeypatch.setenv("COZYQ_VERIFY_DIR", str(tmp_path))
    monkeypatch.setattr(verify, "_KNOWN", {})
    return tmp_path


def test_a_passing_probe_runs_once_and_leaves_no_marker(markers):
    calls = []

    def probe():
        calls.append(1)
        assert (markers / "k.probing").exists()  # armed while it runs
        return verify.Verdict(True, "fine")

    assert verify.verified("k", probe).ok
    assert verify.verified("k", probe).ok
    assert len(calls) == 1
    assert not (markers / "k.probing").exists()


def test_a_probe_that_raises_fails_with_why(markers):
    def probe():
        raise ValueError("shape")

    v = verify.verified("k", probe)
    assert not v.ok and "ValueError: shape" in v.detail
    assert not (markers / "k.probing").exists()


def test_a_marker_left_by_a_dead_probe_is_refused(markers):
    (markers / "k.probing").write_text("pid 1 probing\n")
    ran = []
    v = verify.verified("k", lambda: ran.append(1) or verify.Verdict(True, ""))
    assert not v.ok and verify.CRASHED in v.detail and "k.probing" in v.detail
    assert not ran


def test_a_device_fault_keeps_the_marker_for_the_next_process(markers, monkeypatch):
    v = verify.verified("k", lambda: verify.Verdict(True, "fine"), lambda: "context lost")
    assert not v.ok and "context lost" in v.detail
    assert "context lost" in (markers / "k.probing").read_text()
    monkeypatch.setattr(verify, "_KNOWN", {})  # the next process
    again = verify.verified("k", lambda: verify.Verdict(True, "fine"))
    assert not again.ok and verify.CRASHED in again.detail


def test_library_digest_follows_the_bytes(tmp_path):
    a, b = tmp_path / "a", tmp_path / "b"
    a.write_bytes(b"x" * 3000000)
    b.write_bytes(b"x" * 2999999 + b"y")
    assert verify.library_digest(a) != verify.library_digest(b)
    assert len(verify.library_digest(a)) == 16

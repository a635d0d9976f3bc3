"""The card's self-check on the MI355X: the op library opens only once int8.convrot's and
fp8.rowwise's kernels pass their probes against the float64 law, and a failing probe refuses the
library (it raises; there is no other lane)."""

from __future__ import annotations

import pytest
import torch

from cozyq import prebuilt, verify

pytestmark = pytest.mark.gpu


def test_library_opens_verified():
    ops = prebuilt.library(0)
    assert set(ops.verdicts) == set(verify.PROBES)
    for name, verdict in ops.verdicts.items():
        assert verdict.ok, (name, verdict.detail)
        assert "rel L2" in verdict.detail and "budget" in verdict.detail


@pytest.mark.parametrize("name", sorted(verify.PROBES))
def test_probe_measures_within_budget(name):
    """Each probe run again directly: every case well inside the budget (the kernels round the
    same laws; their error is their output dtype's)."""
    ops = prebuilt.library(0)
    verdict = verify.PROBES[name](torch, ops)
    assert verdict.ok, verdict.detail
    worst = float(verdict.detail.split()[2])
    assert worst < 5e-3, verdict.detail


def test_a_failing_probe_refuses_the_library(monkeypatch, tmp_path):
    """A format whose probe fails makes `library` raise with its detail (the probe here is a
    stand-in that fails; no kernel runs wrongly), and the card is not cached as served."""
    monkeypatch.setenv("COZYQ_VERIFY_DIR", str(tmp_path))
    monkeypatch.setattr(verify, "_KNOWN", {})
    monkeypatch.setattr(prebuilt, "_LIBRARIES", {})
    monkeypatch.setattr(verify, "PROBES", {"int8": lambda torch, ops: verify.Verdict(False, "planted refusal")})
    with pytest.raises(RuntimeError, match="failed their self-check.*int8: planted refusal"):
        prebuilt.library(0)
    assert 0 not in prebuilt._LIBRARIES

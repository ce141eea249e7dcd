"""Host logic of the calibration capture (cdclq.capture): bin planning and file naming
(scripts/capture_hessians.py:73-110)."""
import pytest

from cdclq.capture import accumulator_bytes, out_path_for, plan_bins


def test_plan_bins_first_fit_decreasing_largest_first():
    fam = {"a.down": 96, "a.q": 64, "a.gate": 64, "b.down": 96, "b.q": 64}
    budget = accumulator_bytes(96) + accumulator_bytes(64)
    bins = plan_bins(fam, budget)
    assert bins[0]["owners"][0] == "a.down"  # largest family first, ties by name
    assert all(b["bytes"] <= budget for b in bins)
    assert sorted(o for b in bins for o in b["owners"]) == sorted(fam)
    assert [b["owners"] for b in bins] == [["a.down", "a.gate"], ["b.down", "a.q"], ["b.q"]]


def test_plan_bins_rejects_a_family_above_the_budget():
    with pytest.raises(ValueError, match="a single Hessian at d_in=128"):
        plan_bins({"x": 128}, accumulator_bytes(64))


def test_out_path_for():
    assert out_path_for("h/hess.safetensors", 1, 1) == "h/hess.safetensors"
    assert out_path_for("h/hess.safetensors", 2, 3) == "h/hess.2of3.safetensors"

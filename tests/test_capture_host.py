"""Host logic of the calibration capture (cdclq.capture): the pass plan, the file naming and the
sharing probe (the behaviour of scripts/capture_hessians.py:59-110, :185-208)."""
import pytest

from cdclq.capture import (GIB, SharedInputProbe, device_entry_bytes, pass_file, plan_entry_bytes, plan_passes,
                           human_size)


def test_plan_passes_first_fit_decreasing_largest_first():
    fam = {"a.down": 96, "a.q": 64, "a.gate": 64, "b.down": 96, "b.q": 64}
    budget = plan_entry_bytes(96) + plan_entry_bytes(64)
    passes = plan_passes(fam, budget)
    assert passes[0].owners[0] == "a.down"  # largest input first, ties by name
    assert all(p.planned <= budget for p in passes)
    assert sorted(o for p in passes for o in p.owners) == sorted(fam)
    assert [p.owners for p in passes] == [["a.down", "a.gate"], ["b.down", "a.q"], ["b.q"]]


def test_plan_uses_the_reference_weight_of_four_bytes_per_entry():
    """The same budget splits the same way as the reference (f32 accounting), although the device
    accumulators here are f64: a 4096-wide and a 14336-wide input fit 1 GiB together in one pass."""
    assert plan_entry_bytes(4096) == 4096 * 4096 * 4
    assert len(plan_passes({"q": 4096, "down": 14336}, 1 * GIB)) == 1
    assert device_entry_bytes(4096, paired=False) == 2 * plan_entry_bytes(4096)
    assert device_entry_bytes(4096, paired=True) == 4 * plan_entry_bytes(4096)


def test_plan_passes_rejects_an_owner_above_the_budget():
    with pytest.raises(ValueError, match=r"d_in=128\) needs 64\.0 KiB"):
        plan_passes({"x": 128}, plan_entry_bytes(64))


def test_pass_file():
    assert pass_file("h/hess.safetensors", 1, 1) == "h/hess.safetensors"
    assert pass_file("h/hess.safetensors", 2, 3) == "h/hess.2of3.safetensors"


def test_human_size():
    assert human_size(512) == "0.5 KiB" and human_size(3 << 20) == "3.0 MiB" and human_size(3 * GIB) == "3.00 GiB"


def test_probe_aliases_consecutive_identical_inputs_only():
    """q/k/v read one tensor (aliases of q); o reads another; a later module reading q's tensor
    again after o is its own owner (only the previous input counts)."""
    p = SharedInputProbe()
    a, b = object(), object()
    for name, x in (("q", a), ("k", a), ("v", a), ("o", b), ("late", a)):
        p.hook(name)(None, (x,))
    assert p.alias_of == {"k": "q", "v": "q"}

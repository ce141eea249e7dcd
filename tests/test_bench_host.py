"""bench.py's host-side reporting and contract, on the CPU: the near-midpoint, bits-per-weight and
wall-clock summaries of a step, the reference's row-chunk rule, and the refusal of more than one
GPU (this build measures one)."""
import os
import subprocess
import sys
from types import SimpleNamespace

import pytest

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _stats(bits_codes, bits_total):
    return SimpleNamespace(bits_codes=bits_codes, bits_total=bits_total)


def test_midpoint_report_sums_the_matrices():
    a = dict(code_decisions=10, code_near=1, zero_decisions=4, zero_near=0, cd_decisions=7, cd_near=2)
    b = dict(code_decisions=5, code_near=0, zero_decisions=2, zero_near=1, cd_decisions=3, cd_near=0)
    rep = bench.midpoint_report({"q": (None, a), "k": (None, b)})
    assert rep["per_matrix"] == {"q": a, "k": b}
    assert rep["layer"] == dict(code_decisions=15, code_near=1, zero_decisions=6, zero_near=1, cd_decisions=10,
                                cd_near=2)


def test_bits_per_weight_is_weighted_by_element_count():
    """Config 3's layer: the skeleton gives matrices different bits_total; the layer figure weights
    each by d_out x n (q 2048x2048, k/v 256x2048, o 2048x2048, gate/up 5632x2048, down 2048x5632)."""
    spec = bench.CONFIGS["c3"]
    vals = {"q_proj": 2.5, "k_proj": 3.0, "v_proj": 3.0, "o_proj": 2.5, "gate_proj": 2.75, "up_proj": 2.75,
            "down_proj": 2.625}
    stats = {name: (_stats(2.0, v), None) for name, v in vals.items()}
    rep = bench.bpw_report(spec, stats)
    num = den = 0
    for name, d_out, key in spec["layers"]:
        el = d_out * spec["inputs"][key]
        num += vals[name] * el
        den += el
    assert rep["layer_bits_total"] == round(num / den, 6)
    assert rep["per_matrix"]["down_proj"] == {"bits_codes": 2.0, "bits_total": 2.625}


def test_step_wall_is_additive_and_averaged():
    walls = [{"gram": 1.0, "quantize": 0.5, "chains": {"a": 0.4, "b": 0.5}},
             {"gram": 1.2, "quantize": 0.7, "chains": {"a": 0.6, "b": 0.7}}]
    rep = bench.step_wall_ms(walls)
    assert rep == {"gram": 1100.0, "quantize": 600.0, "chains": {"a": 500.0, "b": 600.0}}
    assert bench.step_wall_ms([{"gram": 0.25, "quantize": 0.5, "chains": {}}]) == {"gram": 250.0, "quantize": 500.0}


@pytest.mark.parametrize("d_out,cfg_rc,nthreads,want", [(4096, 0, 24, 171), (14336, 0, 24, 256), (1024, 0, 24, 43),
                                                        (256, 0, 24, 32), (20, 0, 24, 20), (2048, 64, 24, 64)])
def test_rows_per_chunk_is_the_reference_rule(d_out, cfg_rc, nthreads, want):
    """src/engine.rs:768-770: ceil(d_out / threads) clamped to 32..256 (at most d_out), or the
    configured chunk."""
    spec = {"cfg": {"row_chunk": cfg_rc}, "nthreads": nthreads}
    assert bench.rows_per_chunk(spec, d_out) == want


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "measures one GPU only" in r.stdout

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "cdcl-gptq_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (runs the HIP library through the C ABI)")
    config.addinivalue_line("markers", "slow: longer CPU checks")


def pytest_terminal_summary(terminalreporter):
    """Near-midpoint report of the GPU parity comparisons (the north star asks for every near-midpoint
    rounding decision to be counted and reported): totals over the session, and every comparison in
    which an exemption fired."""
    try:
        from problems import MIDPOINT_LOG
    except ImportError:
        return
    if not MIDPOINT_LOG:
        return
    tot = {}
    both = [r for r in MIDPOINT_LOG if r["oracle"] and r["gpu"]]
    for rec in both:
        for side in ("oracle", "gpu"):
            for k, v in rec[side].items():
                tot[(side, k)] = tot.get((side, k), 0) + v
    fired = [r for r in MIDPOINT_LOG if r["classification"]]
    tr = terminalreporter
    tr.section("near-midpoint report")
    tr.write_line(f"{len(MIDPOINT_LOG)} parity comparisons, {len(both)} with counts from both sides (totalled "
                  f"below); comparisons with an exempt code mismatch: {len(fired)}")
    for side in ("oracle", "gpu"):
        tr.write_line(f"{side}: " + ", ".join(f"{k} {v}" for (s, k), v in sorted(tot.items()) if s == side))
    for r in fired:
        tr.write_line(f"exemption in {r['label']}: {r['classification']}")

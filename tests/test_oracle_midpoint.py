"""Near-midpoint accounting of the parity contract, on the CPU: the oracle's counts and per-element
map, and the classification of code mismatches into exempt (the oracle's own rounding input lies
within 1e-9 of k + 1/2), cascaded (later effects of an exempt one in the same row chunk) and
non-exempt (real differences)."""
import numpy as np

import oracle as O
from problems import classify_mismatches, tie_problem, synth_layer


def tie_cfg(**kw):
    base = dict(bits=4, group=64, block=64, act_order=False, row_chunk=16, passes=2)
    base.update(kw)
    return O.config(**base)


def test_tie_layer_decisions_are_all_near_midpoints():
    """Every phase-1 code and zero point of the tie layer is an exact f32 tie; the map and the counts
    agree (one code decision per element, one zero per row and group of 64 columns)."""
    w, h = tie_problem()
    q = O.quantize_layer(w, h, tie_cfg(method="gptq"), midmap=True)
    mc, mm = q.midpoint, q.midmap
    d_out, n = w.shape
    assert mc["code_decisions"] == d_out * n and mc["zero_decisions"] == d_out * (n // 64)
    assert mc["zero_near"] == d_out * (n // 64)  # -lo / scale = 4.5 in every group
    # every code decision except those clamped either way (k = 10 -> 15 or 16, both 15) is a tie
    assert mc["code_near"] == int((mm & 1).sum()) > 0.85 * d_out * n
    assert int((mm & 4).sum()) == 4 * 64 * mc["zero_near"]
    assert mc["cd_decisions"] == 0 and mc["cd_near"] == 0  # GPTQ: no descent


def test_tie_layer_descent_evaluations_are_counted():
    """With the scales kept (no refit), each descent target w_hat + g / H_jj is w itself (e is a
    power of two, so g = e H_jj and g / H_jj are exact), a tie again."""
    w, h = tie_problem()
    q = O.quantize_layer(w, h, tie_cfg(method="cdcl", refit_scales=False), midmap=True)
    mc, mm = q.midpoint, q.midmap
    assert mc["cd_decisions"] > 0 and mc["cd_near"] > 0
    assert int(((mm & 2) != 0).sum()) <= mc["cd_near"] <= mc["cd_decisions"]


def test_random_layer_has_no_or_few_near_midpoints():
    w, _, h, _ = synth_layer(71, 64, 256, 1000)
    q = O.quantize_layer(w, h, tie_cfg(bits=3, group=128, block=128), midmap=True)
    mc = q.midpoint
    assert mc["code_decisions"] == 64 * 256 and mc["cd_decisions"] > 0
    assert mc["code_near"] + mc["zero_near"] + mc["cd_near"] <= 2  # f32 ties are rare in generic data
    assert int((q.midmap != 0).sum()) <= 2 * 64


def test_classifier_exempts_ties_and_catches_real_differences():
    w, h = tie_problem()
    q = O.quantize_layer(w, h, tie_cfg(method="gptq"), midmap=True)
    # only the code bit: every element of the tie layer also carries its group's zero-point bit
    mm = q.midmap & 1
    near = np.argwhere(mm)
    far = np.argwhere(mm == 0)
    assert near.size and far.size
    rc = 16
    # a tie broken the other way: exempt
    got = q.codes.copy()
    r, c = near[0]
    got[r, c] ^= 1
    assert classify_mismatches(got, q.codes, mm, rc) == dict(mismatches=1, exempt=1, cascaded=0, non_exempt=0, rows=1,
                                                            exempt_chunks=1, chunk_ids=[int(r) // rc])
    # a difference where the oracle's decision was not near a midpoint: non-exempt
    got = q.codes.copy()
    r2, c2 = far[0]
    got[r2, c2] ^= 1
    cls = classify_mismatches(got, q.codes, mm, rc)
    assert cls["non_exempt"] == 1 and cls["exempt"] == 0
    # in the same row chunk as an exempt one it counts as cascaded; in another chunk it does not
    same = [p for p in far if p[0] // rc == r // rc][0]
    other = [p for p in far if p[0] // rc != r // rc][0]
    got = q.codes.copy()
    got[r, c] ^= 1
    got[same[0], same[1]] ^= 1
    assert classify_mismatches(got, q.codes, mm, rc)["cascaded"] == 1
    got[same[0], same[1]] ^= 1
    got[other[0], other[1]] ^= 1
    assert classify_mismatches(got, q.codes, mm, rc)["non_exempt"] == 1


def test_planted_mistakes_are_not_exempt():
    """A real bug (the planted sign error of the in-block compensation) produces mismatches that
    the exemption does not cover."""
    w, _, h, _ = synth_layer(72, 48, 192, 900)
    cfg = tie_cfg(bits=3, group=64, block=64)
    good = O.quantize_layer(w, h, cfg, midmap=True)
    with O.mutation(1):
        bad = O.quantize_layer(w, h, cfg)
    cls = classify_mismatches(bad.codes, good.codes, good.midmap, 16)
    assert cls["mismatches"] > 0 and cls["non_exempt"] > 0

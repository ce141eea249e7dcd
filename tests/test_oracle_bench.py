"""The oracle against the reference's own published benchmark numbers.

tests/golden/readme_bench.json holds the held-out errors printed in the reference README
(README.md:205-241), produced by `cdclq bench` (src/bench.rs) on its synthetic layer. The oracle
regenerates the same inputs (rng.rs stream in src/bench.rs's draw order) and runs RTN, GPTQ and
the CDCL variants (src/bench.rs:209-241), then bench::rel_err on the held-out tokens; every number
must round to the printed digits. This pins, end to end and against the Rust binary's output, the
generator, the matrixmultiply chain GEMMs, the Gram accumulation, the factorisation, phase 1, the
repair and rtn_layer together.
"""
import json
import os

import numpy as np
import pytest

import oracle as O

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "readme_bench.json")))
ARGS = GOLD["args"]
NAMES = {"refit_only": dict(method="cdcl", refine_frac=0.0, cd_sweeps=1, passes=3, refit_scales=1, tol=0.0),
         "cd_only": dict(method="cdcl", refine_frac=1.0, cd_sweeps=1, passes=4, refit_scales=0, tol=0.0),
         "fast": dict(method="cdcl", refine_frac=0.5, cd_sweeps=1, passes=2, refit_scales=1, tol=0.0),
         "balanced": dict(method="cdcl", refine_frac=1.0, cd_sweeps=1, passes=4, refit_scales=1, tol=0.0),
         "default": dict(method="cdcl"), "GPTQ": dict(method="gptq")}


def printed(value: float, text: str) -> bool:
    """value rounds to the printed mantissa digits of text (e.g. '6.195e-3')."""
    mant, ex = text.split("e")
    digits = len(mant.replace(".", "").lstrip("-")) - 1
    return f"{value:.{digits}e}" == f"{float(text):.{digits}e}"


@pytest.fixture(scope="module")
def layer():
    r, n, t, tt = ARGS["rows"], ARGS["cols"], ARGS["tokens"], ARGS["test_tokens"]
    w, x, xte, _, _ = O.bench_inputs(ARGS["seed"], r, n, t, tt)
    h = O.gram_accumulate(x).astype(np.float32)
    return w, x, xte, h


def held_out(layer, cfg, h=None, m=None, xte_t=None):
    w, x, xte, h0 = layer
    q = O.quantize_layer(w, h0 if h is None else h, cfg, m=m, hkey="bench", nthreads=ARGS["nthreads"])
    xt = xte if xte_t is None else xte_t
    return O.rel_err(w, q.dequantize(), xte, xt, w.shape[0], w.shape[1], xte.shape[0]), q


def test_readme_3bit_table(layer):
    """The equal-bits table (README.md:207-219, src/bench.rs:209-241)."""
    tab = GOLD["tables"]["3bit_g128"]
    w, x, xte, h = layer
    rtn = O.rtn_layer(w, O.config(bits=3, act_order=False))
    got = {"RTN": O.rel_err(w, rtn, xte, xte, w.shape[0], w.shape[1], xte.shape[0])}
    for key in ("GPTQ", "refit_only", "cd_only", "fast", "balanced", "default"):
        got[key], _ = held_out(layer, O.config(bits=3, group=128, **NAMES[key]))
    for key, text in tab["held_out"].items():
        assert printed(got[key], text), (key, got[key], text)
    for key, pct in tab["vs_gptq_pct"].items():
        decimals = len(pct.split(".")[1]) if "." in pct else 0
        assert f"{100 * (got[key] / got['GPTQ'] - 1):+.{decimals}f}" == pct, (key, got[key])


@pytest.mark.parametrize("table", ["4bit_g128", "3bit_g128_mse", "2bit_g64", "3bit_skeleton5_8bit"])
def test_readme_configuration_rows(layer, table):
    """README.md:225-236: other bit widths, the MSE grid, group 64, the 5% skeleton."""
    tab = GOLD["tables"][table]
    base = dict(tab["cfg"])
    skel = base.pop("skeleton_pct", 0.0)
    for key, text in tab["held_out"].items():
        kw = dict(base)
        if skel:
            kw.update(skeleton_pct=skel, method="gptq" if key.startswith("GPTQ") else "cdcl")
        else:
            kw.update(NAMES[key])
        v, _ = held_out(layer, O.config(**kw))
        assert printed(v, text), (table, key, v, text)


def test_readme_asymmetric_inputs(layer):
    """README.md:237-239 (src/bench.rs:265-311): noisy inputs, H~ and M from the same stream."""
    tab = GOLD["tables"]["3bit_asym_noise_0.08"]
    r, n, t, tt = ARGS["rows"], ARGS["cols"], ARGS["tokens"], ARGS["test_tokens"]
    w, x, xte, xt, xte_t = O.bench_inputs(ARGS["seed"], r, n, t, tt, tab["asym_noise"])
    ht = O.gram_accumulate(xt).astype(np.float32)
    m = O.gram_accumulate(x, xt).astype(np.float32)
    lay = (w, x, xte, ht)
    runs = {"GPTQ, symmetric target (H~ only)": (O.config(bits=3, method="gptq"), None),
            "GPTQ, asymmetric target (W* = W M H~^-1)": (O.config(bits=3, method="gptq"), m),
            "CDCL-GPTQ, asymmetric target": (O.config(bits=3, method="cdcl"), m)}
    for key, text in tab["held_out"].items():
        cfg, mm = runs[key]
        v, _ = held_out(lay, cfg, h=ht, m=mm, xte_t=xte_t)
        assert printed(v, text), (key, v, text)

"""GPU parity of the evaluation pieces and of the synthetic-benchmark harness (src/engine.rs:808-838,
src/bench.rs): rtn_layer bit-exact against the oracle, rel_err and proxy_loss against the oracle
(the f32 products are the same chains; the f64 sums are parallel on the GPU, tolerance 1e-12),
and `cdclq_bench_run` against the numbers the reference README prints for `cdclq bench`
(tests/golden/readme_bench.json) and against the oracle on a small layer.
"""
import json
import os

import numpy as np
import pytest

import cdclq
import oracle as O

pytestmark = pytest.mark.gpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "readme_bench.json")))
ARGS = GOLD["args"]
README_NAMES = {"RTN": "RTN (no compensation)", "GPTQ": "GPTQ", "refit_only": "ablation: scale refit only (3 passes)",
                "cd_only": "ablation: coordinate descent only (4 passes)",
                "fast": "CDCL-GPTQ fast (50% sub-blocks, 2 passes)",
                "balanced": "CDCL-GPTQ balanced (all sub-blocks, 4 passes)",
                "default": "CDCL-GPTQ default (up to 10 passes, tol 0.001)"}


@pytest.fixture(scope="module")
def ctx():
    c = cdclq.Context(0)
    yield c
    c.close()


def printed(value: float, text: str) -> bool:
    mant, _ = text.split("e")
    digits = len(mant.replace(".", "").lstrip("-")) - 1
    return f"{value:.{digits}e}" == f"{float(text):.{digits}e}"


@pytest.mark.parametrize("bits,group,mse,n", [(3, 128, 0, 300), (4, 64, 1, 256), (2, 0, 0, 200), (8, 32, 1, 96),
                                              (3, 7, 1, 50)])
def test_rtn_matches_oracle(ctx, bits, group, mse, n):
    rng = np.random.default_rng(bits * 100 + n)
    w = (rng.standard_normal((37, n)) * 0.02).astype(np.float32)
    w[3] = 0.0  # an all-zero row takes the [-1, 1] fallback grid
    w[5, :10] = 0.0
    print(f"[bench] rtn bits={bits} group={group} mse={mse} n={n}", flush=True)
    got = cdclq.rtn_layer(ctx, w, cdclq.Config(bits=bits, group=group, mse_grid=bool(mse)))
    ref = O.rtn_layer(w, O.config(bits=bits, group=group, mse_grid=mse))
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_rel_err_and_proxy_loss_match_oracle(ctx):
    rng = np.random.default_rng(7)
    rows, n, t = 48, 320, 700
    w = rng.standard_normal((rows, n)).astype(np.float32)
    wq = (w + 0.01 * rng.standard_normal((rows, n))).astype(np.float32)
    x = rng.standard_normal((t, n)).astype(np.float32)
    xt = (x + 0.05 * rng.standard_normal((t, n))).astype(np.float32)
    for a, b in ((x, x), (x, xt)):
        g = cdclq.rel_err(ctx, w, wq, a, b)
        o = O.rel_err(w, wq, a, b, rows, n, t)
        assert abs(g - o) <= 1e-12 * abs(o), (g, o)
    h = (x.T @ x).astype(np.float32)
    dw, dq, dh = (cdclq.DeviceArray.from_host(ctx, a) for a in (w, wq, h))
    out = cdclq.C.c_double()
    ctx.check(cdclq.lib().cdclq_proxy_loss_device(ctx.ptr, dw.ptr, dq.ptr, rows, n, dh.ptr, cdclq.C.byref(out)))
    ref = O.proxy_loss(w, wq, h)
    assert abs(out.value - ref) <= 1e-9 * abs(ref)
    for a in (dw, dq, dh):
        a.free()


def test_bench_run_reproduces_the_readme_table(ctx):
    """`cdclq bench --rows 512 --cols 2048 --tokens 16384 --test-tokens 4096` (3 bit, group 128):
    every held-out error and percentage the README prints (README.md:207-219)."""
    print("[bench] README 3-bit table", flush=True)
    report, rows = cdclq.bench_run(ctx, cdclq.Config(bits=3, group=128), **ARGS)
    by = {r.name: r for r in rows}
    tab = GOLD["tables"]["3bit_g128"]
    for key, text in tab["held_out"].items():
        assert printed(by[README_NAMES[key]].test, text), (key, by[README_NAMES[key]].test, text)
    base = by["GPTQ"].test
    for key, pct in tab["vs_gptq_pct"].items():
        decimals = len(pct.split(".")[1]) if "." in pct else 0
        assert f"{100 * (by[README_NAMES[key]].test / base - 1):+.{decimals}f}" == pct
    assert report.startswith("## Synthetic layer 512x2048, 16384 calibration tokens, 4096 held-out tokens, 1 threads")
    assert "bits=3 group=128 damp=0.01 act_order=true mse_grid=false sub_block=64 cd_sweeps=1" in report
    assert "### Equal-bits comparison (same grid, ordering, damping)" in report
    assert "| RTN (no compensation) | - | " in report
    assert abs(by["GPTQ"].bpw - (3 + 24 / 128)) < 1e-12


def test_bench_run_reproduces_the_readme_skeleton_and_noise_rows(ctx):
    """README.md:233-239: the 5% 8-bit skeleton and the quantized-input (noise 0.08) experiment."""
    print("[bench] README skeleton + asymmetric rows", flush=True)
    report, rows = cdclq.bench_run(ctx, cdclq.Config(bits=3, group=128, skeleton_pct=5.0, skeleton_bits=8),
                                   asym_noise=0.08, **ARGS)
    by = {r.name: r for r in rows}
    for table in ("3bit_skeleton5_8bit", "3bit_asym_noise_0.08"):
        for name, text in GOLD["tables"][table]["held_out"].items():
            assert printed(by[name].test, text), (name, by[name].test, text)
    assert "### Protected skeleton (5% of input columns at 8 bits) - note the higher bits/weight" in report
    assert "### Quantized-input calibration (relative input noise 0.08): error is ||W x - W_hat x~||" in report
    assert by["GPTQ + skeleton"].bpw > by["GPTQ"].bpw


def test_bench_run_matches_the_oracle_on_a_small_layer(ctx):
    rows_, n, t, tt, seed, noise = 40, 256, 1500, 600, 5, 0.05
    cfg = dict(bits=3, group=64, skeleton_pct=10.0, skeleton_bits=6, block=64)
    print("[bench] small layer vs oracle", flush=True)
    _, rows = cdclq.bench_run(ctx, cdclq.Config(**cfg), rows=rows_, cols=n, tokens=t, test_tokens=tt, seed=seed,
                              asym_noise=noise, nthreads=3)
    by = {r.name: r for r in rows}
    w, x, xte, xt, xte_t = O.bench_inputs(seed, rows_, n, t, tt, noise)
    h = O.gram_accumulate(x).astype(np.float32)
    ncal = min(t, 4096)

    def ev(wq, xc=x, xtc=x, xh=xte, xth=xte):
        return (O.rel_err(w, wq, xc[:ncal], xtc[:ncal], rows_, n, ncal), O.rel_err(w, wq, xh, xth, rows_, n, tt))

    def close(name, loss, errs):
        r = by[name]
        assert abs(r.loss - loss) <= 1e-6 * max(abs(loss), 1e-300), (name, r.loss, loss)
        assert abs(r.calib - errs[0]) <= 1e-12 * errs[0] and abs(r.test - errs[1]) <= 1e-12 * errs[1], name

    base = dict(cfg, skeleton_pct=0.0)
    rtn = O.rtn_layer(w, O.config(**dict(base, act_order=False)))
    close("RTN (no compensation)", 0.0, ev(rtn))
    q = O.quantize_layer(w, h, O.config(**dict(base, method="gptq")), hkey="bench", nthreads=3)
    close("GPTQ", q.stats["loss_final"], ev(q.dequantize()))
    q = O.quantize_layer(w, h, O.config(**dict(base, method="cdcl", refine_frac=0.5, passes=2, tol=0.0)),
                         hkey="bench", nthreads=3)
    close("CDCL-GPTQ fast (50% sub-blocks, 2 passes)", q.stats["loss_final"], ev(q.dequantize()))
    q = O.quantize_layer(w, h, O.config(**dict(cfg, method="cdcl")), hkey="bench", nthreads=3)
    close("CDCL-GPTQ + skeleton", q.stats["loss_final"], ev(q.dequantize()))
    ht = O.gram_accumulate(xt).astype(np.float32)
    m = O.gram_accumulate(x, xt).astype(np.float32)
    q = O.quantize_layer(w, ht, O.config(**dict(base, method="cdcl")), m=m, hkey="bench", nthreads=3)
    close("CDCL-GPTQ, asymmetric target", q.stats["loss_final"], ev(q.dequantize(), x, xt, xte, xte_t))
    floor = by["FP weights on noisy inputs (floor)"]
    fl = ev(w, x, xt, xte, xte_t)
    assert abs(floor.calib - fl[0]) <= 1e-12 * fl[0] and abs(floor.test - fl[1]) <= 1e-12 * fl[1]

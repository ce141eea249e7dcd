"""Writes tests/golden/config_digests.json: the oracle's results for BASELINE configs 2, 3 and 4
at their real shapes, as SHA-256 digests.

    python tests/golden/make_config_digests.py [c2c3] [c4] [c5]    (default: c2c3 c4)

Configs 2 and 3 are the TinyLlama-1.1B-shaped decoder layer (262,144 tokens, 0.5% Student-t(3)
channels); config 4 is the Llama-3-8B-shaped decoder layer (524,288 tokens, 1% outlier channels
x30, n = 4096 and 14336). The oracle needs minutes (c2/c3) to about an hour (c4, on 8 cores) per
layer at these sizes, so it runs here once and the GPU test (tests/test_gpu_configs.py) compares the
engine's outputs with these digests bit for bit. Inputs come from the counter-based generator
(oracle twins of the device generator: same seeds as bench.py's CONFIGS), so the GPU regenerates
identical bytes. Config 4's tokens are generated and accumulated in slabs of 16384 tokens (eight of
the Gram's 2048-token chunks; the f64 accumulation over chunks is the same sequence as one call).

Recorded per config: the SHA-256 of each input's H (f32, the cast of the f64 Gram) and, per matrix,
of codes, scales, zeros (f32 bytes), perm (u32) and gbits, plus the LayerStats fields. Config 4
also records each input's f64 H, the oracle's near-midpoint counts per matrix, and the SHA-256 of
U = upper_chol_of_inverse(H + 0.01 mean(diag H) I) (f32, the public linalg entry point,
src/linalg.rs:362-375) of its n = 14336 input.

Config 5 (Llama-3-70B MLP, n = 8192 and 28672, H~ = X~^T X~ and M = X^T X~ over 524,288 tokens,
asymmetric target) records the f32 and f64 digests of both inputs' H~ and M (about 3 hours of the
oracle's Gram on 8 cores) and, per matrix, the digests of its first C5_CHUNKS row chunks (default
7, the chunk size of the full run), with those rows' own stats and near-midpoint counts.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "tests")]

import numpy as np  # noqa: E402

import bench  # noqa: E402  (config table and seeds only)
import oracle as O  # noqa: E402

OUT = os.path.join(HERE, "config_digests.json")
SLAB = 16384  # tokens generated and accumulated at a time (a multiple of the Gram's 2048-token chunk)


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def channel_args(spec: dict, i: int, n: int):
    """(ch_scale, heavy) of input i: the oracle twins of bench.channel_spec."""
    cseed = bench.input_seeds(i)[0]
    xg = spec.get("xgen")
    if xg is None:
        return O.synth_outlier_scales(cseed, n, spec["outlier_frac"], spec["outlier_factor"]), None
    if xg["kind"] == "lognormal":
        return O.synth_lognormal_scales(cseed, n, xg["sigma"]), None
    assert xg["kind"] == "heavy"
    return None, (O.synth_outlier_scales(cseed, n, xg["frac"], 2.0) != 1.0).astype(np.uint8)


def hessian64(spec: dict, i: int, n: int):
    """f64 Gram of input i over the config's tokens, generated and accumulated slab by slab. With
    the asymmetric target (X~ = X + sigma N(0, 1), the perturbation stream indexed by element):
    (H~ = X~^T X~, M = X^T X~); otherwise H = X^T X."""
    _, tseed, pseed = bench.input_seeds(i)
    cs, heavy = channel_args(spec, i, n)
    T = spec["tokens"]
    asym = spec.get("asym_noise", 0.0)
    h = np.zeros((n, n), np.float64)
    m = np.zeros((n, n), np.float64) if asym else None
    t0 = time.time()
    for r0 in range(0, T, SLAB):
        t = min(SLAB, T - r0)
        x = O.synth_tokens(tseed, t, n, cs, row0=r0, heavy=heavy)
        if asym:
            xt = x + O.synth_normal(pseed, t * n, asym, offset=r0 * n).reshape(t, n)
            O.gram_accumulate(xt, h=h)
            O.gram_accumulate(x, xt, h=m)
            del xt
        else:
            O.gram_accumulate(x, h=h)
        del x
        if (r0 // SLAB) % 8 == 7:
            print(f"  n={n}: {r0 + SLAB}/{T} tokens, {time.time() - t0:.0f}s", flush=True)
    return (h, m) if asym else h


def hessians(spec: dict) -> dict:
    """key -> (H64, H32) of every input."""
    hs = {}
    for i, (key, n) in enumerate(spec["inputs"].items()):
        t0 = time.time()
        h64 = hessian64(spec, i, n)
        hs[key] = (h64, h64.astype(np.float32))
        print(f"{key}: H {n}x{n} in {time.time() - t0:.1f}s", flush=True)
    return hs


STAT_FIELDS = ("loss_gptq", "loss_final", "subblocks_total", "subblocks_refined", "code_updates", "skeleton_groups",
               "bits_codes", "bits_total")


def run_config(name: str, hs: dict, midpoints: bool = False) -> dict:
    spec = bench.CONFIGS[name]
    out = {"workload": spec["workload"], "tokens": spec["tokens"], "cfg": spec["cfg"], "nthreads": spec["nthreads"],
           "inputs": {key: {"n": n, "h32_sha256": sha(hs[key][1])} for key, n in spec["inputs"].items()},
           "layers": {}}
    if midpoints:
        for key in spec["inputs"]:
            out["inputs"][key]["h64_sha256"] = sha(hs[key][0])
    cfg = O.config(**spec["cfg"])
    cache = O.Cache()  # one PrepCache for the layer, as the reference pipeline (src/pipeline.rs:117)
    for li, (lname, d_out, key) in enumerate(spec["layers"]):
        n = spec["inputs"][key]
        w = O.synth_normal(bench.weight_seed(li), d_out * n, spec["wsigma"]).reshape(d_out, n)
        t0 = time.time()
        q = O.quantize_layer(w, hs[key][1], cfg, hkey=key, cache=cache, nthreads=spec["nthreads"])
        st = q.stats
        rec = {
            "d_out": d_out, "n": n, "input": key,
            "codes": sha(q.codes), "scales": sha(q.scales), "zeros": sha(q.zeros), "perm": sha(q.perm),
            "gbits": sha(q.gbits),
            "stats": {f: st[f] for f in STAT_FIELDS},
        }
        if midpoints:
            rec["midpoint"] = q.midpoint
        out["layers"][lname] = rec
        print(f"{name} {lname} {d_out}x{n}: {time.time() - t0:.1f}s loss_final {st['loss_final']:.6e} "
              f"updates {st['code_updates']} midpoint {q.midpoint}", flush=True)
    return out


def factor_digest(h64: np.ndarray) -> str:
    """SHA-256 of U (f32) for H + 0.01 mean(diag H) I, the damping bench and the GPU test apply."""
    h = h64.copy()
    n = h.shape[0]
    h[np.arange(n), np.arange(n)] += 0.01 * np.mean(np.diag(h))
    t0 = time.time()
    u = O.upper_chol_of_inverse(h)
    print(f"U {n}x{n} in {time.time() - t0:.1f}s", flush=True)
    return sha(u)


def run_config5(chunks: int) -> dict:
    """Config 5 (Llama-3-70B MLP, asymmetric target): the full-size H~ and M of both inputs, then
    the first `chunks` row chunks of every matrix (the chunk size of the full run, passed
    explicitly): rows are quantized in independent chunks, and the permutation and the target
    W* = ((W M') U^T) U act row by row, so these rows equal the same rows of the full run."""
    name = "c5"
    spec = bench.CONFIGS[name]
    out = {"workload": spec["workload"], "tokens": spec["tokens"], "cfg": spec["cfg"], "nthreads": spec["nthreads"],
           "inputs": {}, "layers": {}}
    hs = {}
    for i, (key, n) in enumerate(spec["inputs"].items()):
        t0 = time.time()
        h64, m64 = hessian64(spec, i, n)
        hs[key] = (h64.astype(np.float32), m64.astype(np.float32))
        out["inputs"][key] = {"n": n, "h32_sha256": sha(hs[key][0]), "m32_sha256": sha(hs[key][1]),
                              "h64_sha256": sha(h64), "m64_sha256": sha(m64)}
        del h64, m64
        print(f"{key}: H~ and M {n}x{n} in {time.time() - t0:.1f}s", flush=True)
    cache = O.Cache()
    for li, (lname, d_out, key) in enumerate(spec["layers"]):
        n = spec["inputs"][key]
        rc = bench.rows_per_chunk(spec, d_out)
        rows = min(d_out, chunks * rc)
        w = O.synth_normal(bench.weight_seed(li), rows * n, spec["wsigma"]).reshape(rows, n)
        cfg = O.config(**{**spec["cfg"], "row_chunk": rc})
        t0 = time.time()
        q = O.quantize_layer(w, hs[key][0], cfg, m=hs[key][1], hkey=key, cache=cache, nthreads=spec["nthreads"])
        out["layers"][lname] = {
            "d_out": d_out, "n": n, "input": key, "rows": rows, "row_chunk": rc,
            "codes": sha(q.codes), "scales": sha(q.scales), "zeros": sha(q.zeros), "perm": sha(q.perm),
            "gbits": sha(q.gbits), "rows_stats": {f: q.stats[f] for f in STAT_FIELDS}, "rows_midpoint": q.midpoint,
        }
        print(f"{name} {lname} first {rows} of {d_out} rows x {n}: {time.time() - t0:.1f}s "
              f"loss_final {q.stats['loss_final']:.6e} updates {q.stats['code_updates']}", flush=True)
    return out


def load() -> dict:
    if os.path.exists(OUT):
        with open(OUT) as f:
            return json.load(f)
    return {"generator": "tests/golden/make_config_digests.py (oracle/cdclq_oracle.c)", "configs": {}}


def save(res: dict):
    with open(OUT, "w") as f:
        json.dump(res, f, indent=1, sort_keys=True)
    print("wrote", OUT, flush=True)


def main(argv):
    O.set_threads(int(os.environ.get("ORACLE_THREADS", os.cpu_count() or 8)))
    which = argv or ["c2c3", "c4"]
    res = load()
    if "c2c3" in which:
        c2, c3 = bench.CONFIGS["c2"], bench.CONFIGS["c3"]
        assert (c2["inputs"], c2["tokens"], c2["xgen"]) == (c3["inputs"], c3["tokens"], c3["xgen"])
        hs = hessians(c2)
        for c in ("c2", "c3"):
            res["configs"][c] = run_config(c, hs)
        save(res)
    if "c4" in which:
        hs = hessians(bench.CONFIGS["c4"])
        rec = run_config("c4", hs, midpoints=True)
        rec["inputs"]["mlp_act"]["u32_sha256"] = factor_digest(hs["mlp_act"][0])
        res["configs"]["c4"] = rec
        save(res)
    if "c5" in which:
        rec = run_config5(chunks=int(os.environ.get("C5_CHUNKS", "7")))
        res = load()  # another run may have written meanwhile
        res["configs"]["c5"] = rec
        save(res)


if __name__ == "__main__":
    main(sys.argv[1:])

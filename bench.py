#!/usr/bin/env python3
"""Benchmark of the MI355X engine on BASELINE.json's headline metric:
seconds per Llama-3-8B-shaped decoder layer (config 4: H-accumulation + U + GPTQ + repair).

One step = one full decoder layer: 4 Hessian accumulations over 524,288 synthetic tokens (the
inputs of q/k/v, o, gate/up and down) and 7 quantize_layer calls (INT4, g128, B128, act-order,
damp 0.01, repair on with the reference defaults), with the factor cache shared by q/k/v and by
gate/up as in the reference pipeline. Inputs (X, W) are generated in HBM before the timed region.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c1|c2|c3|c4|c5] [--serial]
                    [--no-cpu-baseline] [--profile-gram] [--workload layer|container] [--floor-rows R]

Prints one JSON line (rank 0). The CPU baseline is the C restatement of the reference (oracle/)
timed on bounded samples of the same step on this host and scaled to the step (see `sample`).
"""
from __future__ import annotations

import argparse
import concurrent.futures
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "cdcl-gptq_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import numpy as np  # noqa: E402

FP32_PEAK_TFLOPS = 157.3  # MI355X dense FP32 matrix peak (AMD published)

CONFIGS = {
    # Llama-3-8B-shaped decoder layer
    "c4": dict(
        workload="llama3-8b decoder layer (BASELINE config 4)",
        tokens=256 * 2048,
        inputs={"attn_in": 4096, "attn_out": 4096, "mlp_in": 4096, "mlp_act": 14336},
        layers=[("q_proj", 4096, "attn_in"), ("k_proj", 1024, "attn_in"), ("v_proj", 1024, "attn_in"),
                ("o_proj", 4096, "attn_out"), ("gate_proj", 14336, "mlp_in"), ("up_proj", 14336, "mlp_in"),
                ("down_proj", 4096, "mlp_act")],
        wsigma=0.015, outlier_frac=0.01, outlier_factor=30.0,
        cfg=dict(bits=4, group=128, block=128, damp=0.01, act_order=True),
        nthreads=24,
    ),
    # TinyLlama-1.1B-shaped decoder layer, INT3 g128, act-order, repair
    # (reference defaults: passes 10, tol 1e-3); 0.5% Student-t(3) channels
    "c2": dict(
        workload="tinyllama-1.1b decoder layer (BASELINE config 2)",
        tokens=128 * 2048,
        inputs={"attn_in": 2048, "attn_out": 2048, "mlp_in": 2048, "mlp_act": 5632},
        layers=[("q_proj", 2048, "attn_in"), ("k_proj", 256, "attn_in"), ("v_proj", 256, "attn_in"),
                ("o_proj", 2048, "attn_out"), ("gate_proj", 5632, "mlp_in"), ("up_proj", 5632, "mlp_in"),
                ("down_proj", 2048, "mlp_act")],
        wsigma=0.02, xgen=dict(kind="heavy", frac=0.005),
        cfg=dict(bits=3, group=128, block=128, act_order=True),
        nthreads=24,
    ),
    # the same layer at INT2 g64, MSE grid, passes 8, 5% INT8 skeleton
    # (the saliency permutation depends on W, so every matrix has its own factorisation)
    "c3": dict(
        workload="tinyllama-1.1b decoder layer, INT2 + 5% INT8 skeleton (BASELINE config 3)",
        tokens=128 * 2048,
        inputs={"attn_in": 2048, "attn_out": 2048, "mlp_in": 2048, "mlp_act": 5632},
        layers=[("q_proj", 2048, "attn_in"), ("k_proj", 256, "attn_in"), ("v_proj", 256, "attn_in"),
                ("o_proj", 2048, "attn_out"), ("gate_proj", 5632, "mlp_in"), ("up_proj", 5632, "mlp_in"),
                ("down_proj", 2048, "mlp_act")],
        wsigma=0.02, xgen=dict(kind="heavy", frac=0.005),
        cfg=dict(bits=2, group=64, block=128, act_order=True, mse_grid=True, passes=8, skeleton_pct=5.0,
                 skeleton_bits=8),
        nthreads=24,
    ),
    # Llama-3-70B-shaped MLP, INT3 g128, passes 6, asymmetric target
    # W* = W M H~^-1 with H~ = X~^T X~, M = X^T X~, X~ = X + N(0, 0.05^2); log-normal channel scales
    "c5": dict(
        workload="llama3-70b MLP (BASELINE config 5)",
        tokens=128 * 4096,
        inputs={"mlp_in": 8192, "mlp_act": 28672},
        layers=[("gate_proj", 28672, "mlp_in"), ("up_proj", 28672, "mlp_in"), ("down_proj", 8192, "mlp_act")],
        wsigma=0.01, xgen=dict(kind="lognormal", sigma=0.5), asym_noise=0.05,
        cfg=dict(bits=3, group=128, block=128, act_order=True, passes=6),
        nthreads=24,
    ),
    # single 2048x2048 layer (CPU-runnable reference case)
    "c1": dict(
        workload="single 2048x2048 layer (BASELINE config 1)",
        tokens=4096,
        inputs={"x": 2048},
        layers=[("linear", 2048, "x")],
        wsigma=0.02, outlier_frac=0.01, outlier_factor=20.0,
        cfg=dict(bits=4, group=128, block=128, damp=0.01, act_order=False, passes=4, tol=1e-6, row_chunk=64),
        nthreads=24,
    ),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def input_seeds(i: int):
    """(channel pick / scale seed, token seed, perturbation seed) of the config's i-th input."""
    return 1000 + 7 * i, 2000 + 7 * i, 4000 + 7 * i


def weight_seed(li: int) -> int:
    return 3000 + li


def channel_spec(spec: dict, i: int, n: int):
    """(channel scales or None, Student-t channel mask or None) of input i, host arrays."""
    import cdclq

    cseed = input_seeds(i)[0]
    xg = spec.get("xgen")
    if xg is None:
        return cdclq.synth_outlier_scales(cseed, n, spec["outlier_frac"], spec["outlier_factor"]), None
    if xg["kind"] == "heavy":
        return None, cdclq.synth_heavy_channels(cseed, n, xg["frac"])
    if xg["kind"] == "lognormal":
        return cdclq.synth_lognormal_scales(cseed, n, xg["sigma"]), None
    raise ValueError(xg["kind"])


def make_inputs(ctx, spec: dict, only=None):
    """Token-major calibration inputs in HBM: {key: X} and, for the asymmetric target, {key: X~}.
    `only`: a subset of the input keys (each keeps its own seeds)."""
    import cdclq

    T = spec["tokens"]
    xs, xts = {}, {}
    for i, (key, n) in enumerate(spec["inputs"].items()):
        if only is not None and key not in only:
            continue
        cs, heavy = channel_spec(spec, i, n)
        xs[key] = cdclq.DeviceArray(ctx, (T, n), np.float32)
        cdclq.synth_tokens_device(ctx, input_seeds(i)[1], T, n, xs[key], ch_scale=cs, heavy=heavy)
        if spec.get("asym_noise"):
            xts[key] = cdclq.DeviceArray(ctx, (T, n), np.float32)
            cdclq.synth_perturb_device(ctx, input_seeds(i)[2], xs[key], xts[key], spec["asym_noise"])
    return xs, xts


def gram_jobs(spec: dict, xs: dict, xts: dict, h64s: dict, m64s: dict):
    """The layer's accumulations as (x, y, h, input key): H = X^T X per input, or, with the
    asymmetric target, H~ = X~^T X~ and M = X^T X~."""
    jobs = []
    for key in xs:
        if xts:
            jobs += [(xts[key], xts[key], h64s[key], key), (xs[key], xts[key], m64s[key], key)]
        else:
            jobs.append((xs[key], xs[key], h64s[key], key))
    return jobs


class LayerStep:
    """One decoder layer of a config, resident in HBM, and its step.

    Holds the calibration inputs (generated on the device), the f64 accumulators and their f32
    copies (H, and M with the asymmetric target), the weights and the output buffers. A step runs
    every accumulation in one batched launch, then one quantize_layer call per matrix. The matrices
    form one chain per input: the matrices of an input share its factorisation through one
    context's factor cache, in the reference's order (src/pipeline.rs:109-130); different inputs
    are independent, so with serial=False their chains run concurrently, each on its own context
    (stream, workspace, cache) from its own host thread. Each call is the same synchronous
    quantize_layer as in the serial order, with the same results. Every cache is cleared at the
    start of a step (each step's H are new)."""

    def __init__(self, ctx, spec: dict, serial: bool = False, weights: bool = True):
        import cdclq

        self.ctx, self.spec, self.serial = ctx, spec, serial
        self.T = spec["tokens"]
        self.xs, self.xts = make_inputs(ctx, spec)
        self.h64s, self.h32s, self.m64s, self.m32s = {}, {}, {}, {}
        for key, n in spec["inputs"].items():
            self.h64s[key] = cdclq.DeviceArray(ctx, (n, n), np.float64)
            self.h32s[key] = cdclq.DeviceArray(ctx, (n, n), np.float32)
            if self.xts:
                self.m64s[key] = cdclq.DeviceArray(ctx, (n, n), np.float64)
                self.m32s[key] = cdclq.DeviceArray(ctx, (n, n), np.float32)
        self.jobs = gram_jobs(spec, self.xs, self.xts, self.h64s, self.m64s)
        self.cfg = cdclq.Config(**spec["cfg"])
        self.ws, self.outs, self.perm_gbits = {}, {}, {}
        self.chains, self.chain_ctx, self.pool = {}, {}, None
        if not weights:
            return
        for li, (name, d_out, key) in enumerate(spec["layers"]):
            n = spec["inputs"][key]
            self.ws[name] = cdclq.DeviceArray(ctx, (d_out, n), np.float32)
            ctx.check(cdclq.lib().cdclq_synth_normal_device(ctx.ptr, weight_seed(li), 0, d_out * n, spec["wsigma"],
                                                             self.ws[name].ptr))
            ng = (n + self.cfg.group - 1) // self.cfg.group
            self.outs[name] = (cdclq.DeviceArray(ctx, (d_out, n), np.uint8),
                               cdclq.DeviceArray(ctx, (d_out, ng), np.float32),
                               cdclq.DeviceArray(ctx, (d_out, ng), np.float32))
        for name, d_out, key in spec["layers"]:
            self.chains.setdefault(key, []).append((name, d_out, key))
        self.chain_ctx = {k: (ctx if serial else cdclq.Context(0)) for k in self.chains}
        if not serial:
            self.pool = concurrent.futures.ThreadPoolExecutor(max_workers=len(self.chains))

    def contexts(self) -> list:
        return [self.ctx] + ([] if self.serial else list(self.chain_ctx.values()))

    def gram(self, keys):
        """The accumulations of the inputs `keys` in one launch (each equals its own
        gram_accumulate), then their f32 copies."""
        import cdclq

        ctx, T = self.ctx, self.T
        js = [j for j in self.jobs if j[3] in keys]
        for _, _, h, _ in js:
            h.zero()
        cdclq.gram_accumulate_batch_device(ctx, [j[0] for j in js], [j[1] for j in js], [T] * len(js),
                                           [j[0].shape[1] for j in js], [j[2] for j in js])
        for key in keys:
            n = self.spec["inputs"][key]
            ctx.check(cdclq.lib().cdclq_f64_to_f32_device(ctx.ptr, self.h64s[key].ptr, n * n, self.h32s[key].ptr))
            if self.xts:
                ctx.check(cdclq.lib().cdclq_f64_to_f32_device(ctx.ptr, self.m64s[key].ptr, n * n,
                                                               self.m32s[key].ptr))

    def run_chain(self, cctx, names):
        """The chain's quantize_layer calls in order on one context; returns ({name: (LayerStats,
        near-midpoint counts)}, seconds)."""
        import cdclq

        out = {}
        t0 = time.perf_counter()
        for name, d_out, key in names:
            n = self.spec["inputs"][key]
            c, s, z = self.outs[name]
            perm, gbits, st = cdclq.quantize_layer_device(cctx, self.ws[name], d_out, n, self.h32s[key],
                                                          self.m32s.get(key), key, self.cfg, c, s, z,
                                                          nthreads=self.spec["nthreads"])
            out[name] = (st, cctx.last_midpoint_counts())
            self.perm_gbits[name] = (perm, gbits)
        return out, time.perf_counter() - t0

    def step(self):
        """One layer: returns ({name: (LayerStats, near-midpoint counts)}, host wall split)."""
        stats = {}
        for c in set(self.chain_ctx.values()):
            c.clear_cache()
        t0 = time.perf_counter()
        self.gram(list(self.spec["inputs"]))  # all accumulations in one launch (synchronous)
        t1 = time.perf_counter()
        chain_s = {}
        if self.serial:  # the matrices one after another
            res, _ = self.run_chain(self.ctx, self.spec["layers"])
            stats.update(res)
        else:  # the chains at once, each on its own context
            futs = {k: self.pool.submit(self.run_chain, self.chain_ctx[k], self.chains[k]) for k in self.chains}
            for k, fut in futs.items():
                res, chain_s[k] = fut.result()
                stats.update(res)
        return stats, {"gram": t1 - t0, "quantize": time.perf_counter() - t1, "chains": chain_s}

    def free_inputs(self):
        for d in list(self.xs.values()) + list(self.xts.values()):
            d.free()
        self.xs, self.xts = {}, {}

    def close_chains(self):
        if self.pool is not None:
            self.pool.shutdown()
            self.pool = None
            for c in self.chain_ctx.values():
                c.close()
            self.chain_ctx = {k: self.ctx for k in self.chain_ctx}

    def free(self):
        self.close_chains()
        self.free_inputs()
        for d in (list(self.h64s.values()) + list(self.h32s.values()) + list(self.m64s.values())
                  + list(self.m32s.values()) + list(self.ws.values()) + [a for o in self.outs.values() for a in o]):
            d.free()


def gram_flops(n: int, t: int) -> float:
    """Algorithmic work of one symmetric H accumulation: n(n+1) t flops (one triangle)."""
    return float(n) * (n + 1) * t


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or the platform string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or platform.machine()


def factorisations(spec: dict) -> list:
    """Widths of the distinct factorisations of one step: one per input (the factor cache is keyed
    by input and permutation, src/engine.rs:718), or one per matrix when the skeleton makes the
    permutation depend on W."""
    if spec["cfg"].get("skeleton_pct", 0.0) > 0.0:
        return [spec["inputs"][key] for _, _, key in spec["layers"]]
    return list(spec["inputs"].values())


def rows_per_chunk(spec: dict, d_out: int) -> int:
    """The reference's row chunk (src/engine.rs:768-770) at the config's thread count."""
    rc = spec["cfg"].get("row_chunk", 0)
    if rc <= 0:
        rc = min(max(-(-d_out // spec["nthreads"]), 32), 256)
    return max(min(rc, d_out), 1)


FACTOR_SAMPLE_MAX_N = 16384  # wider factorisations are extrapolated by n^3 (minutes on the host)


def cpu_baseline(spec: dict, cores: int, fetch) -> dict:
    """The oracle (C restatement of the reference's rayon path) timed on bounded samples of the
    step's own work, on this host, then scaled to one step.

    `fetch(kind, key_or_name, rows)` returns the workload's own host arrays after the timed region:
    ("h", key) the f32 H, ("m", key) the f32 M, ("w", name, rows) the first rows of a matrix.
    * Gram: each distinct width accumulates a slab of synthetic tokens of that width (the work
      does not depend on the values); scaled by T / slab (2048-token chunks in sequence, each the
      same work) per accumulation.
    * Factorisation + phase 1 + 2: for each distinct width, the widest-row matrix of that width is
      quantized on one wave of row chunks (one chunk per thread, the reference's chunk size, with
      the step's real H and W rows): secs_prepare is the factorisation, secs_quant the wave of
      chunks. Each matrix is then ceil(chunks / threads) waves of its own chunk size (per-chunk time
      taken linear in its rows), which is how chunks map to the reference's thread pool.
    * Widths above FACTOR_SAMPLE_MAX_N (config 5's 28672) take the sample of the widest width at
      or below it, scaled by n^3 (factor) and n^2 x rows (chunks, target GEMMs)."""
    import oracle as O

    O.set_threads(cores)
    T = spec["tokens"]
    asym = bool(spec.get("asym_noise"))
    njobs = 2 if asym else 1  # H~ and M per input with the asymmetric target
    widths = sorted(set(spec["inputs"].values()))
    notes = []
    gram_full = 0.0
    for n in widths:
        # long enough that the per-call setup (the n x n chunk buffer) is amortised as in a whole
        # run: a single 2048-token chunk at n = 14336 takes 0.68 s against 0.61 s per chunk of 8192
        slab = min(T, 32768 if n <= 4096 else 8192 if n <= 16384 else 2048)
        x = O.synth_tokens(102, slab, n, None)
        t0 = time.perf_counter()
        O.gram_accumulate(x)
        t = time.perf_counter() - t0
        del x
        cnt = sum(1 for v in spec["inputs"].values() if v == n)
        gram_full += t * njobs * cnt * T / slab
        notes.append(f"gram {slab} tokens at n={n} {t:.2f}s")
    cfg = O.config(**spec["cfg"])
    samples = {}  # width -> (factor s, per-row chunk s, target s per row)
    for n in [v for v in widths if v <= FACTOR_SAMPLE_MAX_N]:
        key = next(k for k, v in spec["inputs"].items() if v == n)
        name, d_out, _ = max((l for l in spec["layers"] if spec["inputs"][l[2]] == n), key=lambda l: l[1])
        rc = rows_per_chunk(spec, d_out)
        chunks = min(cores, -(-d_out // rc))
        rows = min(d_out, chunks * rc)
        h = fetch("h", key)
        m = fetch("m", key) if asym else None
        w = fetch("w", name, rows)
        c = O.config(**{**spec["cfg"], "row_chunk": rc})
        if asym:  # the target GEMMs are inside secs_prepare: time the factor on its own
            q = O.quantize_layer(w, h, c, m=m, hkey=key, nthreads=cores)
            hd = h.astype(np.float64)
            hd[np.arange(n), np.arange(n)] += cfg.damp * np.mean(np.diag(hd))
            t0 = time.perf_counter()
            O.upper_chol_of_inverse(hd)
            t_fac = time.perf_counter() - t0
            t_tgt = max(0.0, q.stats["secs_prepare"] - t_fac) / rows
        else:
            q = O.quantize_layer(w, h, c, hkey=key, nthreads=cores)
            t_fac, t_tgt = q.stats["secs_prepare"], 0.0
        samples[n] = (t_fac, q.stats["secs_quant"] / rc, t_tgt)
        notes.append(f"{name} n={n}: factor {t_fac:.2f}s, one wave of {chunks} chunks x {rc} rows "
                     f"{q.stats['secs_quant']:.2f}s")
        del h, m, w
    fac_full = quant_full = target_full = 0.0
    for n in factorisations(spec):
        n0 = max(v for v in samples if v <= n) if any(v <= n for v in samples) else max(samples)
        fac_full += samples[n0][0] * (n / n0) ** 3
    per_matrix = {}
    for name, d_out, key in spec["layers"]:
        n = spec["inputs"][key]
        n0 = n if n in samples else max(samples)
        rc = rows_per_chunk(spec, d_out)
        waves = -(-(-(-d_out // rc)) // cores)
        per_matrix[name] = samples[n0][1] * rc * waves * (n / n0) ** 2
        quant_full += per_matrix[name]
        target_full += samples[n0][2] * d_out * (n / n0) ** 2
    total = gram_full + fac_full + quant_full + target_full
    sample = (f"oracle on {cores} threads of {cpu_model()}, timed in this run (Gram on synthetic tokens of each "
              "width; factorisation and row chunks on the step's own H and W rows): "
              + "; ".join(notes) + ". Scaled to the step: Gram by tokens, each matrix by its waves of row chunks "
              "(chunk time linear in rows); factorisations measured at their width"
              + (" (wider ones by n^3)" if any(v > FACTOR_SAMPLE_MAX_N for v in widths) else "")
              + ". Repair passes are data-dependent per chunk, so the waves are a model of the full step.")
    out = {"value": round(total, 2), "unit": "s/layer", "cores": cores, "kind": "port", "cpu": cpu_model(),
           "sample": sample}
    chk = recorded_quant_check(spec)
    if chk is not None:
        out["value_with_quant_check"] = round(total - quant_full * (1.0 - chk), 2)
        out["quant_check"] = (f"whole matrices measured {chk} of the chunk-wave model for phase 1 + 2 "
                              f"(profiles/cpu_baseline_{spec.get('name', '')}.md)")
    return {**out, "phases_s": {"gram": round(gram_full, 2), "factor": round(fac_full, 2),
                                           "quant": round(quant_full, 2), "target": round(target_full, 2)},
            "quant_s_per_matrix": {k: round(v, 2) for k, v in per_matrix.items()}}


def recorded_quant_check(spec: dict):
    """The measured / modelled phase 1 + 2 ratio recorded by `bench.py --cpu-validate` runs in
    profiles/cpu_baseline_<config>.md (None if not recorded)."""
    path = os.path.join(ROOT, "profiles", f"cpu_baseline_{spec.get('name', '')}.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("quant_measured_over_model:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_validate(spec: dict, cores: int, fetch, name: str) -> dict:
    """Checks the CPU baseline's chunk-wave model on one whole matrix: the oracle quantizes every
    row of `name` (its own H and W from the step, the config's row chunks) and its measured phase
    1 + 2 time is set beside the model's prediction for that matrix."""
    import oracle as O

    model = cpu_baseline(spec, cores, fetch)
    _, d_out, key = next(l for l in spec["layers"] if l[0] == name)
    h = fetch("h", key)
    w = fetch("w", name, d_out)
    cfg = O.config(**{**spec["cfg"], "row_chunk": rows_per_chunk(spec, d_out)})
    q = O.quantize_layer(w, h, cfg, hkey=key, nthreads=cores)
    pred = model["quant_s_per_matrix"][name]
    return {"cpu_validate": name, "threads": cores, "cpu": cpu_model(), "rows": d_out, "n": spec["inputs"][key],
            "measured_quant_s": round(q.stats["secs_quant"], 2), "predicted_quant_s": round(pred, 2),
            "measured_over_predicted": round(q.stats["secs_quant"] / pred, 3),
            "measured_factor_s": round(q.stats["secs_prepare"], 2), "model": model}


def recorded_traffic(summary: str):
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3 --pmc summary
    profiles/<summary>.md (FETCH_SIZE + WRITE_SIZE, calibrated against a copy of known size);
    None if not recorded."""
    path = os.path.join(ROOT, "profiles", f"{summary}.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def profile_gram(ctx, spec, jobs):
    """One calibration copy of known size, then one batched gram launch (for rocprofv3 --pmc)."""
    import ctypes
    import cdclq
    nbytes = 1 << 30
    src = cdclq.DeviceArray(ctx, (nbytes // 4,), np.float32)
    dst = cdclq.DeviceArray(ctx, (nbytes // 4,), np.float32)
    src.zero()
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    rc = hip.hipMemcpy(dst.ptr, src.ptr, nbytes, 3)  # hipMemcpyDeviceToDevice: one copy kernel
    if rc != 0 or hip.hipDeviceSynchronize() != 0:
        raise RuntimeError(f"calibration copy failed ({rc})")
    for _, _, h, _ in jobs:
        h.zero()
    T = spec["tokens"]
    cdclq.gram_accumulate_batch_device(ctx, [j[0] for j in jobs], [j[1] for j in jobs], [T] * len(jobs),
                                       [j[0].shape[1] for j in jobs], [j[2] for j in jobs])
    x_bytes = sum(T * j[0].shape[1] * 4 * (1 if j[0] is j[1] else 2) for j in jobs)
    h_bytes = sum(j[0].shape[1] ** 2 * 8 for j in jobs)
    print(json.dumps({"profile": "gram", "workload": spec["workload"], "calibration_copy_bytes": nbytes,
                      "algorithmic_read_bytes": x_bytes + h_bytes, "algorithmic_write_bytes": h_bytes}), flush=True)


HBM_PEAK_GBS = 8000.0  # MI355X HBM3E (AMD published)

DATA_DESC = {
    "outlier": "synthetic (counter-based N(0,1) activations with outlier channels, N(0,s^2) weights)",
    "heavy": "synthetic (counter-based N(0,1) activations with Student-t(3) channels, N(0,s^2) weights)",
    "lognormal": "synthetic (counter-based N(0,1) activations with log-normal channel scales, X~ = X + N(0,0.05^2), "
                 "N(0,s^2) weights)",
}


def container_layers(spec):
    """(name, d_out, d_in) of the layer's quantized matrices."""
    return [(name, d_out, spec["inputs"][key]) for name, d_out, key in spec["layers"]]


def container_inputs(spec, seed=77):
    """Synthetic engine outputs of one layer in the engine's form: 4-bit codes, f16-exact scales,
    integer zero points, a random act-order permutation, group 128 (what quantize_layer writes)."""
    rng = np.random.default_rng(seed)
    g, bits = spec["cfg"]["group"], spec["cfg"]["bits"]
    out = {}
    for name, d_out, n in container_layers(spec):
        ng = (n + g - 1) // g
        codes = rng.integers(0, 1 << bits, (d_out, n), dtype=np.uint8)
        scales = rng.uniform(2e-4, 2e-2, (d_out, ng)).astype(np.float16).astype(np.float32)
        zeros = rng.integers(0, 1 << bits, (d_out, ng)).astype(np.float32)
        perm = rng.permutation(n).astype(np.uint32)
        out[name] = (codes, scales, zeros, perm, np.full(ng, bits, np.uint8))
    return out


def container_bytes(d_out, n, g, bits, out_bytes=2):
    """Algorithmic HBM bytes of one dequantization launch: packed rows, f16 scales and u8 zeros
    read once, the output written once, plus the per-column map (8 B per column)."""
    ng = (n + g - 1) // g
    rb = (n * bits + 7) // 8
    return d_out * rb + d_out * ng * 3 + d_out * n * out_bytes + 8 * n


def container_bench(args, spec):
    import cdclq

    ctx = cdclq.Context(0)
    L = cdclq.lib()
    g, bits = spec["cfg"]["group"], spec["cfg"]["bits"]
    host = container_inputs(spec)
    dev = {}
    for name, d_out, n in container_layers(spec):
        codes, scales, zeros, perm, gbits = host[name]
        ng = gbits.size
        rb = cdclq.row_bytes(n, g, gbits)
        dev[name] = dict(
            codes=cdclq.DeviceArray.from_host(ctx, codes), scales=cdclq.DeviceArray.from_host(ctx, scales),
            zeros=cdclq.DeviceArray.from_host(ctx, zeros), perm=cdclq.DeviceArray.from_host(ctx, perm),
            gbits=gbits, rb=rb, qw=cdclq.DeviceArray(ctx, (d_out, rb), np.uint8),
            s16=cdclq.DeviceArray(ctx, (d_out, ng), np.uint16), qz=cdclq.DeviceArray(ctx, (d_out, ng), np.uint8),
            p32=cdclq.DeviceArray(ctx, (n,), np.int32), out=cdclq.DeviceArray(ctx, (d_out, n), np.uint16))

    def step():
        for name, d_out, n in container_layers(spec):
            d = dev[name]
            ng = d["gbits"].size
            ctx.check(L.cdclq_pack_layer_device(ctx.ptr, d_out, n, g, d["gbits"].ctypes.data, ng, d["codes"].ptr,
                                                d["scales"].ptr, d["zeros"].ptr, d["perm"].ptr, d["qw"].ptr,
                                                d_out * d["rb"], d["s16"].ptr, d["qz"].ptr, d["p32"].ptr))
            ctx.check(L.cdclq_dequantize_packed_device(ctx.ptr, d_out, n, g, d["gbits"].ctypes.data, ng, d["qw"].ptr,
                                                       d_out * d["rb"], d["s16"].ptr, d["qz"].ptr, d["p32"].ptr,
                                                       cdclq.DTYPE_BF16, d["out"].ptr))

    if args.profile:
        # counter-collection run: 1 GiB device-to-device copy (byte-counter calibration), one step
        import ctypes
        hip = ctypes.CDLL("libamdhip64.so")
        nb = 1 << 30
        a, b = cdclq.DeviceArray(ctx, (nb,), np.uint8), cdclq.DeviceArray(ctx, (nb,), np.uint8)
        assert hip.hipMemcpy(b.ptr, a.ptr, ctypes.c_size_t(nb), 3) == 0
        assert hip.hipDeviceSynchronize() == 0
        step()
        print(json.dumps({"profile": "container", "copy_bytes": nb}), flush=True)
        ctx.close()
        return
    for i in range(args.warmup):
        step()
    ctx.set_timing(True)
    ctx.reset_timing()
    times = []
    for i in range(args.steps):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
        log(f"[bench] container step {i} {times[-1] * 1e3:.3f} ms")
    ph = ctx.timing()
    ctx.set_timing(False)
    ms_per_step = 1000.0 * sum(times) / len(times)
    byts = args.steps * sum(container_bytes(d_out, n, g, bits) for _, d_out, n in container_layers(spec))
    pack_bytes = args.steps * sum(d_out * n + d_out * ((n * bits + 7) // 8) + d_out * ((n + g - 1) // g) * 11
                                  for _, d_out, n in container_layers(spec))
    dq_ms, pk_ms = ph["dequant"]["ms"], ph["pack"]["ms"]
    achieved = byts / (dq_ms * 1e-3) / 1e9 if dq_ms > 0 else 0.0
    log(f"[bench] device ms per step: pack {pk_ms / args.steps:.3f} dequant {dq_ms / args.steps:.3f}")
    result = {
        "metric": "sec per Llama-3-8B-shaped layer: pack to cdclq-v1 + dequantize to bf16 (7 matrices)",
        "value": round(ms_per_step / 1000.0, 6),
        "unit": "s/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic engine outputs (4-bit codes, f16 scales, integer zeros, random act-order perm)",
        "config": {"workload": "llama3-8b decoder layer container (" + spec["workload"] + ")",
                   "layers": {name: [d_out, n] for name, d_out, n in container_layers(spec)},
                   "bits": bits, "group": g, "out_dtype": "bf16", "parallelism": "1 GPU"},
        "phases_ms_per_step": {"pack": round(pk_ms / args.steps, 4), "dequant": round(dq_ms / args.steps, 4)},
        "roofline": {
            "bound": "hbm",
            "kernel": "k_dequant_rows (packed rows -> bf16, original column order)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": recorded_traffic("dequant_container_traffic"),
            "traffic_unit": "bytes per launch, mean over the 7 launches (profiles/dequant_container_traffic.md)",
            "launches": ph["dequant"]["launches"],
            "pack_kernels_gbs": round(pack_bytes / (pk_ms * 1e-3) / 1e9, 1) if pk_ms > 0 else None,
        },
    }
    if not args.no_cpu_baseline:
        import oracle as O

        cores = min(os.cpu_count() or 1, 16)
        O.set_threads(cores)
        name, d_out, n = container_layers(spec)[0]
        codes, scales, zeros, perm, gbits = host[name]
        t0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - t0 < 10.0 or reps == 0:
            qw, s16, qz, p32 = O.pack_layer(codes, scales, zeros, perm, gbits, g)
            O.dequantize_packed(qw, s16, qz, p32, gbits, g, "BF16")
            reps += 1
        t_one = (time.perf_counter() - t0) / reps
        total = sum(do * nn for _, do, nn in container_layers(spec))
        result["cpu_baseline"] = {
            "value": round(t_one * total / (d_out * n), 4), "unit": "s/layer", "cores": cores, "kind": "port",
            "sample": f"oracle pack_layer + dequantize_packed (BF16) of {name} ({d_out}x{n}), {reps} reps, "
                      f"scaled by element count to the layer's 7 matrices"}
    print(json.dumps(result), flush=True)
    ctx.close()


def step_wall_ms(walls: list) -> dict:
    """Host wall-clock split of the timed steps (means): the accumulations, then the quantize calls
    (with the chains concurrent: from the first chain's start to the last one's end, and each
    chain's own span). gram + quantize is the step; the per-phase device times overlap instead."""
    k = len(walls)
    out = {"gram": round(1e3 * sum(w["gram"] for w in walls) / k, 2),
           "quantize": round(1e3 * sum(w["quantize"] for w in walls) / k, 2)}
    if walls[0]["chains"]:
        out["chains"] = {c: round(1e3 * sum(w["chains"][c] for w in walls) / k, 2) for c in walls[0]["chains"]}
    return out


def midpoint_report(stats: dict) -> dict:
    """Near-midpoint rounding decisions of the step (cdclq_ctx_last_midpoint_counts after each
    call): per matrix and summed over the layer. A decision is near when the f64 quotient of its
    f32 operands lies within 1e-9 of k + 1/2 and the two candidates differ after clamping."""
    per = {name: mid for name, (_, mid) in stats.items()}
    tot = {}
    for mid in per.values():
        for f, v in mid.items():
            tot[f] = tot.get(f, 0) + v
    return {"layer": tot, "per_matrix": per}


def bpw_report(spec: dict, stats: dict) -> dict:
    """Effective bits per weight (LayerStats.bits_total: codes plus the f16 scale and 8-bit zero
    point of each group, src/quant.rs:248-250) per matrix and weighted by element count over the
    layer."""
    per, num, den = {}, 0.0, 0
    for name, d_out, key in spec["layers"]:
        st = stats[name][0]
        per[name] = {"bits_codes": st.bits_codes, "bits_total": st.bits_total}
        num += st.bits_total * d_out * spec["inputs"][key]
        den += d_out * spec["inputs"][key]
    return {"layer_bits_total": round(num / den, 6), "per_matrix": per}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--config", default="c4", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-gram", action="store_true",
                    help="counter-collection run: one 1 GiB device-to-device copy (calibration of the HBM "
                         "byte counters), then one launch of the dominant kernel on this config's inputs")
    ap.add_argument("--workload", default="layer", choices=["layer", "container"],
                    help="layer: the headline quantization step; container: pack + dequantize of the "
                         "layer's quantized matrices (cdclq-v1)")
    ap.add_argument("--profile", action="store_true",
                    help="with --workload container: counter-collection run (1 GiB copy + one step)")
    ap.add_argument("--serial", action="store_true",
                    help="quantize the layer's matrices one after another on one context (default: the chains "
                         "of matrices that share an input run concurrently, one context each)")
    ap.add_argument("--cpu-validate", default="",
                    help="after the timed steps, quantize every row of this matrix on the CPU oracle and print "
                         "its time beside the CPU baseline model's prediction (instead of the bench line)")
    ap.add_argument("--floor-rows", type=int, default=0,
                    help="latency-floor run (under a kernel trace): the config's matrices cut to their first "
                         "FLOOR_ROWS rows, same inputs and settings, one untimed step; prints the phase times")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print(f"bench.py: this build measures one GPU only (requested --gpus {args.gpus}, WORLD_SIZE {world}); "
              "sharding the path over several GPUs is a design only, not run here.", flush=True)
        sys.exit(2)

    import cdclq

    spec = dict(CONFIGS[args.config], name=args.config)
    if args.floor_rows > 0:
        # the same matrices with fewer rows in flight: each sweep launch then runs its rows'
        # dependent chains with no other waves on their SIMDs
        spec = dict(spec, layers=[(name, min(d_out, args.floor_rows), key) for name, d_out, key in spec["layers"]])
        args.steps, args.warmup, args.no_cpu_baseline, args.serial = 1, 0, True, True
    if args.workload == "container":
        container_bench(args, spec)
        return
    T = spec["tokens"]
    ctx = cdclq.Context(0)
    log(f"[bench] {spec['workload']}: generating inputs in HBM")
    if args.profile_gram:
        L = LayerStep(ctx, spec, serial=True, weights=False)
        profile_gram(ctx, spec, L.jobs)
        ctx.close()
        return
    L = LayerStep(ctx, spec, serial=args.serial)
    jobs, all_ctx, cfg = L.jobs, L.contexts(), L.cfg
    step = L.step
    for i in range(args.warmup):
        t0 = time.perf_counter()
        step()
        log(f"[bench] warmup {i} {time.perf_counter() - t0:.3f}s")
    for c in all_ctx:
        c.set_timing(True)
        c.reset_timing()
    times, walls = [], []
    for i in range(args.steps):
        t0 = time.perf_counter()
        stats, wall = step()
        times.append(time.perf_counter() - t0)
        walls.append(wall)
        log(f"[bench] step {i} {times[-1]:.3f}s (gram {wall['gram']:.3f}s, quantize {wall['quantize']:.3f}s)")
    ph = {}
    for c in all_ctx:  # device time per phase, summed over the contexts (concurrent chains overlap)
        for k, v in c.timing().items():
            e = ph.setdefault(k, {"ms": 0.0, "launches": 0})
            e["ms"] += v["ms"]
            e["launches"] += v["launches"]
        c.set_timing(False)
    ms_per_step = 1000.0 * sum(times) / len(times)
    for name, (st, mid) in stats.items():
        log(f"[bench] {name}: loss_gptq {st.loss_gptq:.6e} loss_final {st.loss_final:.6e} "
            f"updates {st.code_updates} prepare {st.secs_prepare:.3f}s quant {st.secs_quant:.3f}s near-midpoint {mid}")
    gram_ms = ph["gram"]["ms"]
    gram_launches = ph["gram"]["launches"]
    # algorithmic work, one launch for all of the step's accumulations: n(n+1)T per symmetric H (one
    # triangle), 2 n^2 T per cross-covariance
    flops = args.steps * sum(gram_flops(j[0].shape[1], T) if j[0] is j[1] else 2.0 * j[0].shape[1] ** 2 * T
                             for j in jobs)
    achieved = flops / (gram_ms * 1e-3) / 1e12 if gram_ms > 0 else 0.0
    phases = {k: round(v["ms"] / args.steps, 3) for k, v in ph.items()}
    log(f"[bench] device ms per step by phase: {phases}")
    L.close_chains()
    if args.floor_rows > 0:
        print(json.dumps({"profile": "floor-rows", "workload": spec["workload"], "rows": args.floor_rows,
                          "layers": {name: [d_out, spec["inputs"][key]] for name, d_out, key in spec["layers"]},
                          "phases_ms": phases}), flush=True)
        ctx.close()
        return
    result = {
        "metric": "sec per Llama-3-8B-shaped layer (H-accum+U+GPTQ+repair); MFMA util, HBM GB/s"
        if args.config == "c4" else f"sec per layer ({spec['workload']})",
        "value": round(ms_per_step / 1000.0, 4),
        "unit": "s/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 2),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32+f64",
        "data": DATA_DESC[(spec.get("xgen") or {"kind": "outlier"})["kind"]],
        "config": {"workload": spec["workload"], "tokens": T,
                   "layers": {name: [d_out, spec["inputs"][key]] for name, d_out, key in spec["layers"]},
                   "quant": {**spec["cfg"], "passes": cfg.passes, "tol": cfg.tol}, "parallelism": "1 GPU",
                   "schedule": "matrices one after another" if args.serial else
                   "one chain of matrices per input, chains concurrent (one context and stream each)"},
        "step_wall_ms": step_wall_ms(walls),
        ("phases_ms_per_step" if args.serial else "device_ms_per_step_summed_over_contexts"): phases,
        "near_midpoint": midpoint_report(stats),
        "bits_per_weight": bpw_report(spec, stats),
        "matrices": {name: {"loss_gptq": st.loss_gptq, "loss_final": st.loss_final, "code_updates": st.code_updates}
                     for name, (st, _) in stats.items()},
        "roofline": {
            "bound": "mfma",
            "kernel": f"k_gram_dma (the step's {len(jobs)} accumulations H += X^T Y in "
                      f"{gram_launches // max(args.steps, 1)} launch(es), K=1 f32 MFMA chains, f64 chunks)",
            "achieved": round(achieved, 2),
            "peak": FP32_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / FP32_PEAK_TFLOPS, 4),
            "traffic": recorded_traffic(f"gram_{args.config}_traffic"),
            "traffic_unit": f"bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                            f"profiles/gram_{args.config}_traffic.md)",
            "launches": gram_launches,
        },
    }
    if not args.no_cpu_baseline:
        cores = min(os.cpu_count() or 1, 16)
        log(f"[bench] timing the CPU baseline sample on {cores} threads")

        def fetch(kind, what, rows=None):
            if kind == "w":
                return L.ws[what].download()[:rows]
            return (L.h32s if kind == "h" else L.m32s)[what].download()

        L.free_inputs()
        if args.cpu_validate:
            print(json.dumps(cpu_validate(spec, cores, fetch, args.cpu_validate)), flush=True)
            ctx.close()
            return
        result["cpu_baseline"] = cpu_baseline(spec, cores, fetch)
    print(json.dumps(result), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()

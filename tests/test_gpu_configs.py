"""The BASELINE configurations at their real shapes on the GPU.

Configs 2 and 3 (TinyLlama-1.1B-shaped layer, 262,144 tokens with 0.5% Student-t(3) channels):
bit for bit against the oracle. The oracle needs minutes per layer at this size, so its results
are committed as SHA-256 digests (tests/golden/config_digests.json, written by
tests/golden/make_config_digests.py from the oracle's twins of the counter-based generator). The
test regenerates the same inputs on the device, accumulates H on the device (its digest pins the
full-size Gram), and compares every matrix's codes, scales, zeros, perm and group widths with the
digests and its LayerStats with the oracle's (losses within 1e-6 relative, counts exact). A
mismatching matrix is re-run through the oracle here, which names the first differing element.

Config 4 (Llama-3-8B layer, 524,288 tokens, n = 4096 and 14336), the headline benchmark, runs
through bench.LayerStep with its chains concurrent, as bench.py times it, and is compared with the
oracle's digests in the same way, including each matrix's near-midpoint counts and U of the
n = 14336 input. The concurrent schedule is also checked on config 2's layer over two steps.

Config 5 (Llama-3-70B MLP: n = 28672 H~ and M over 524,288 tokens, asymmetric target): the full-size
H~ and M and the first row chunks of every matrix against the oracle's digests (the oracle cannot
run every row of this layer here in reasonable time; chunks are independent), and the whole layer
through size-independent properties: two runs bit-identical, codes on the grid, f16-exact positive
scales, integer zero points, a permutation, repair never raising the loss, and the factor: U upper
triangular with a positive diagonal and U^T U H x = x.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import bench
import cdclq
import oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config_digests.json")


@pytest.fixture(scope="module")
def ctx():
    c = cdclq.Context(0)
    yield c
    c.close()


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def device_hessians(ctx, spec, only=None):
    """H32 (and M32 with the asymmetric target) of the config's inputs (or the keys in `only`),
    generated and accumulated on the device in one launch; also returns the f64 accumulators."""
    xs, xts = bench.make_inputs(ctx, spec, only)
    T = spec["tokens"]
    keys = {k: n for k, n in spec["inputs"].items() if k in xs}
    h64s = {k: cdclq.DeviceArray(ctx, (n, n), np.float64) for k, n in keys.items()}
    m64s = {k: cdclq.DeviceArray(ctx, (n, n), np.float64) for k, n in keys.items()} if xts else {}
    jobs = bench.gram_jobs(spec, xs, xts, h64s, m64s)
    for _, _, h, _ in jobs:
        h.zero()
    cdclq.gram_accumulate_batch_device(ctx, [j[0] for j in jobs], [j[1] for j in jobs], [T] * len(jobs),
                                       [j[0].shape[1] for j in jobs], [j[2] for j in jobs])
    for d in list(xs.values()) + list(xts.values()):
        d.free()

    def to32(d64, n):
        d32 = cdclq.DeviceArray(ctx, (n, n), np.float32)
        ctx.check(cdclq.lib().cdclq_f64_to_f32_device(ctx.ptr, d64.ptr, n * n, d32.ptr))
        return d32

    h32s = {k: to32(h64s[k], n) for k, n in keys.items()}
    m32s = {k: to32(m64s[k], n) for k, n in keys.items()} if xts else {}
    return h32s, m32s, h64s, m64s


def quantize(ctx, spec, li, h32, m32=None, key="layer"):
    name, d_out, k = spec["layers"][li]
    n = spec["inputs"][k]
    w = cdclq.DeviceArray(ctx, (d_out, n), np.float32)
    ctx.check(cdclq.lib().cdclq_synth_normal_device(ctx.ptr, bench.weight_seed(li), 0, d_out * n, spec["wsigma"],
                                                     w.ptr))
    cfg = cdclq.Config(**spec["cfg"])
    ng = (n + cfg.group - 1) // cfg.group
    c = cdclq.DeviceArray(ctx, (d_out, n), np.uint8)
    s = cdclq.DeviceArray(ctx, (d_out, ng), np.float32)
    z = cdclq.DeviceArray(ctx, (d_out, ng), np.float32)
    perm, gbits, st = cdclq.quantize_layer_device(ctx, w, d_out, n, h32, m32, key, cfg, c, s, z,
                                                  nthreads=spec["nthreads"])
    out = dict(perm=perm, gbits=gbits, stats=st, codes=c.download(), scales=s.download(), zeros=z.download())
    for a in (w, c, s, z):
        a.free()
    return out


def assert_properties(r, bits, label):
    c, sc, z, p, st = r["codes"], r["scales"], r["zeros"], r["perm"], r["stats"]
    maxq = (1 << bits) - 1
    assert np.array_equal(np.sort(p), np.arange(p.size)), f"{label}: perm is not a permutation"
    assert int(c.max()) <= maxq and np.all(r["gbits"] == bits), f"{label}: code outside the {bits}-bit grid"
    assert np.all(sc > 0) and np.array_equal(sc.astype(np.float16).astype(np.float32), sc), f"{label}: scales"
    assert np.all((z >= 0) & (z <= maxq) & (z == np.round(z))), f"{label}: zero points"
    assert 0 < st.loss_final <= st.loss_gptq, f"{label}: loss_final {st.loss_final} > loss_gptq {st.loss_gptq}"


def assert_same_run(a, b, label):
    for f in ("perm", "gbits", "codes", "zeros"):
        assert np.array_equal(a[f], b[f]), f"{label}: {f} differs between two runs"
    assert np.array_equal(a["scales"].view(np.uint32), b["scales"].view(np.uint32)), f"{label}: scales differ"
    assert a["stats"].loss_final == b["stats"].loss_final and a["stats"].code_updates == b["stats"].code_updates


def check_factor(ctx, h64_dev, n, label, probes=2):
    """U of the damped H (src/linalg.rs:362-375 with the engine's relative damping): upper
    triangular, positive diagonal, U^T U H v = v on random probes (f64 products in row blocks)."""
    h = h64_dev.download()
    h[np.arange(n), np.arange(n)] += 0.01 * np.mean(np.diag(h))
    u = cdclq.upper_chol_of_inverse(h, n, ctx)
    assert not np.any(np.tril(u, -1)) and np.all(np.diag(u) > 0), f"{label}: U not upper / diagonal not positive"
    rng = np.random.default_rng(7)
    blk = 2048
    for _ in range(probes):
        v = rng.standard_normal(n)
        hv = h @ v
        uhv = np.concatenate([u[i:i + blk].astype(np.float64) @ hv for i in range(0, n, blk)])
        back = np.zeros(n)
        for i in range(0, n, blk):
            back += u[i:i + blk].astype(np.float64).T @ uhv[i:i + blk]
        err = np.linalg.norm(back - v) / np.linalg.norm(v)
        print(f"[configs] {label}: |U^T U H v - v| / |v| = {err:.2e}", flush=True)
        assert err <= 5e-3, f"{label}: U^T U H v - v relative error {err:.2e}"


# ---------------------------------------------------------------- configs 2 and 3 vs the oracle
@pytest.mark.parametrize("cname", ["c2", "c3"])
def test_tinyllama_configs_match_the_oracle(ctx, cname):
    spec = bench.CONFIGS[cname]
    with open(GOLDEN) as f:
        gold = json.load(f)["configs"][cname]
    print(f"[configs] {cname}: {spec['workload']}, T={spec['tokens']}", flush=True)
    h32s, _, h64s, _ = device_hessians(ctx, spec)
    hosts = {}
    for key, n in spec["inputs"].items():
        hosts[key] = h32s[key].download()
        assert sha(hosts[key]) == gold["inputs"][key]["h32_sha256"], f"{cname} {key}: H differs from the oracle's"
        h64s[key].free()
    ctx.clear_cache()  # one PrepCache for the layer (src/pipeline.rs:117), as the digests were made
    for li, (name, d_out, key) in enumerate(spec["layers"]):
        print(f"[configs] {cname} {name} {d_out}x{spec['inputs'][key]}", flush=True)
        r = quantize(ctx, spec, li, h32s[key], key=key)
        g = gold["layers"][name]
        same = all(sha(r[f]) == g[f] for f in ("codes", "scales", "zeros", "perm", "gbits"))
        if not same:  # locate the first difference with the oracle itself (minutes at this size)
            n = spec["inputs"][key]
            w = O.synth_normal(bench.weight_seed(li), d_out * n, spec["wsigma"]).reshape(d_out, n)
            qo = O.quantize_layer(w, hosts[key], O.config(**spec["cfg"]), hkey=key, nthreads=spec["nthreads"])
            bad = np.argwhere(r["codes"] != qo.codes)
            where = f"first code mismatch at {bad[0].tolist()} of {len(bad)}" if bad.size else "codes equal"
            raise AssertionError(f"{cname} {name}: outputs differ from the oracle's digests ({where}; perm equal: "
                                 f"{np.array_equal(r['perm'], qo.perm)}, scales equal: "
                                 f"{np.array_equal(r['scales'], qo.scales)})")
        st = r["stats"]
        for f in ("loss_gptq", "loss_final"):
            a, b = getattr(st, f), g["stats"][f]
            assert abs(a - b) <= 1e-6 * abs(b), f"{cname} {name}: {f} {a!r} vs oracle {b!r}"
        for f in ("subblocks_total", "subblocks_refined", "code_updates", "skeleton_groups", "bits_codes",
                  "bits_total"):
            assert getattr(st, f) == g["stats"][f], f"{cname} {name}: {f} {getattr(st, f)} vs {g['stats'][f]}"
    for d in h32s.values():
        d.free()


def compare_with_digests(cname, gold, name, codes, scales, zeros, perm, gbits, st, mid=None):
    got = dict(codes=codes, scales=scales, zeros=zeros, perm=perm, gbits=gbits)
    g = gold["layers"][name]
    diff = [f for f in ("codes", "scales", "zeros", "perm", "gbits") if sha(got[f]) != g[f]]
    assert not diff, f"{cname} {name}: {diff} differ from the oracle's digests"
    for f in ("loss_gptq", "loss_final"):
        a, b = getattr(st, f), g["stats"][f]
        assert abs(a - b) <= 1e-6 * abs(b), f"{cname} {name}: {f} {a!r} vs oracle {b!r}"
    for f in ("subblocks_total", "subblocks_refined", "code_updates", "skeleton_groups", "bits_codes", "bits_total"):
        assert getattr(st, f) == g["stats"][f], f"{cname} {name}: {f} {getattr(st, f)} vs {g['stats'][f]}"
    if mid is not None and "midpoint" in g:
        assert mid == g["midpoint"], f"{cname} {name}: near-midpoint counts {mid} vs oracle {g['midpoint']}"


def test_concurrent_chains_match_the_oracle(ctx):
    """The schedule behind the headline number (bench.py's LayerStep, serial=False): config 2's
    layer with one chain per input (q->k->v, o, gate->up, down), the four chains concurrent on their
    own contexts from their own host threads after one batched accumulation launch. Two steps in a
    row (each clears the factor caches); every matrix equals the oracle's digests."""
    spec = bench.CONFIGS["c2"]
    with open(GOLDEN) as f:
        gold = json.load(f)["configs"]["c2"]
    L = bench.LayerStep(ctx, spec, serial=False)
    try:
        for rep in range(2):
            print(f"[configs] c2 concurrent chains, step {rep}", flush=True)
            stats, wall = L.step()
            print(f"[configs] step {rep}: gram {wall['gram']:.3f}s quantize {wall['quantize']:.3f}s "
                  f"chains {wall['chains']}", flush=True)
            for key in spec["inputs"]:
                assert sha(L.h32s[key].download()) == gold["inputs"][key]["h32_sha256"], f"c2 {key}: H differs"
            for name, _, _ in spec["layers"]:
                c, s, z = L.outs[name]
                perm, gbits = L.perm_gbits[name]
                st, mid = stats[name]
                compare_with_digests("c2", gold, name, c.download(), s.download(), z.download(), perm, gbits, st,
                                     mid)
    finally:
        L.free()


# ---------------------------------------------------------------- config 5 at full size
def test_config5_first_chunks_match_the_oracle(ctx):
    """Config 5 (Llama-3-70B MLP, asymmetric target) through bench.LayerStep with its chains
    concurrent: both inputs' H~ and M (f32 and f64, n = 8192 and 28672, 524,288 tokens) equal the
    oracle's, and so do the permutation, group widths and the codes, scales and zeros of each
    matrix's first row chunks (the oracle ran those rows only, with the full run's chunk size: row
    chunks are independent and the target W* = ((W M') U^T) U is row-wise)."""
    spec = bench.CONFIGS["c5"]
    with open(GOLDEN) as f:
        gold = json.load(f)["configs"].get("c5")
    if gold is None:
        pytest.skip("no config 5 digests recorded (tests/golden/make_config_digests.py c5)")
    print(f"[configs] c5: {spec['workload']}, T={spec['tokens']}, chains concurrent", flush=True)
    L = bench.LayerStep(ctx, spec, serial=False)
    try:
        stats, wall = L.step()
        print(f"[configs] c5 step: gram {wall['gram']:.3f}s quantize {wall['quantize']:.3f}s", flush=True)
        L.free_inputs()
        for key in spec["inputs"]:
            g = gold["inputs"][key]
            for label, dev in (("h32", L.h32s[key]), ("m32", L.m32s[key]), ("h64", L.h64s[key]), ("m64", L.m64s[key])):
                assert sha(dev.download()) == g[f"{label}_sha256"], f"c5 {key}: {label} differs from the oracle's"
        for name, d_out, key in spec["layers"]:
            g = gold["layers"][name]
            rows = g["rows"]
            assert g["row_chunk"] == bench.rows_per_chunk(spec, d_out)
            c, s, z = L.outs[name]
            perm, gbits = L.perm_gbits[name]
            got = dict(codes=c.download()[:rows], scales=s.download()[:rows], zeros=z.download()[:rows], perm=perm,
                       gbits=gbits)
            diff = [f for f in ("codes", "scales", "zeros", "perm", "gbits") if sha(got[f]) != g[f]]
            st = stats[name][0]
            print(f"[configs] c5 {name}: first {rows} of {d_out} rows, loss_final {st.loss_final:.6e} "
                  f"updates {st.code_updates}", flush=True)
            assert not diff, f"c5 {name}: {diff} of the first {rows} rows differ from the oracle's digests"
    finally:
        L.free()



def test_config5_full_size_properties(ctx):
    """Llama-3-70B MLP: gate_proj 28672 x 8192 and down_proj 8192 x 28672, INT3 g128, passes 6, with
    the asymmetric target from H~ and M accumulated on the device over 524,288 tokens (X with
    log-normal channel scales, X~ = X + N(0, 0.05^2)); the n = 28672 factor checked directly."""
    spec = bench.CONFIGS["c5"]
    bits = spec["cfg"]["bits"]
    for key, li in (("mlp_in", 0), ("mlp_act", 2)):
        n = spec["inputs"][key]
        print(f"[configs] c5 {key}: H~ and M at n={n}, T={spec['tokens']}", flush=True)
        h32s, m32s, h64s, m64s = device_hessians(ctx, spec, only=[key])
        name, d_out, _ = spec["layers"][li]
        runs = []
        for rep in range(2):
            ctx.clear_cache()
            print(f"[configs] c5 {name} {d_out}x{n} run {rep}", flush=True)
            runs.append(quantize(ctx, spec, li, h32s[key], m32s[key], key=key))
        assert_same_run(runs[0], runs[1], f"c5 {name}")
        assert_properties(runs[0], bits, f"c5 {name}")
        st = runs[0]["stats"]
        print(f"[configs] c5 {name}: loss_gptq {st.loss_gptq:.6e} loss_final {st.loss_final:.6e} "
              f"updates {st.code_updates}", flush=True)
        m64s[key].free()
        for d in (h32s[key], m32s[key]):
            d.free()
        if key == "mlp_act":
            check_factor(ctx, h64s[key], n, "c5 H~ n=28672")
        h64s[key].free()


def test_config4_layer_matches_the_oracle(ctx):
    """Config 4 at full size, the headline benchmark's own layer and schedule (bench.LayerStep with
    the chains concurrent): every input's H (f32 and f64) and every matrix's codes, scales, zeros,
    perm, gbits, LayerStats and near-midpoint counts equal the oracle's digests, and U of the
    n = 14336 input through the public upper_chol_of_inverse equals the oracle's U."""
    spec = bench.CONFIGS["c4"]
    with open(GOLDEN) as f:
        gold = json.load(f)["configs"].get("c4")
    if gold is None:
        pytest.skip("no config 4 digests recorded (tests/golden/make_config_digests.py c4)")
    print(f"[configs] c4: {spec['workload']}, T={spec['tokens']}, chains concurrent", flush=True)
    L = bench.LayerStep(ctx, spec, serial=False)
    try:
        stats, wall = L.step()
        print(f"[configs] c4 step: gram {wall['gram']:.3f}s quantize {wall['quantize']:.3f}s", flush=True)
        L.free_inputs()
        for key in spec["inputs"]:
            g = gold["inputs"][key]
            assert sha(L.h32s[key].download()) == g["h32_sha256"], f"c4 {key}: H (f32) differs from the oracle's"
            assert sha(L.h64s[key].download()) == g["h64_sha256"], f"c4 {key}: H (f64) differs from the oracle's"
        for name, _, _ in spec["layers"]:
            c, s, z = L.outs[name]
            perm, gbits = L.perm_gbits[name]
            st, mid = stats[name]
            print(f"[configs] c4 {name}: loss_final {st.loss_final:.6e} updates {st.code_updates} near {mid}",
                  flush=True)
            compare_with_digests("c4", gold, name, c.download(), s.download(), z.download(), perm, gbits, st, mid)
        n = spec["inputs"]["mlp_act"]
        h = L.h64s["mlp_act"].download()
        h[np.arange(n), np.arange(n)] += 0.01 * np.mean(np.diag(h))
        u = cdclq.upper_chol_of_inverse(h, n, ctx)
        assert sha(u) == gold["inputs"]["mlp_act"]["u32_sha256"], "c4 n=14336: U differs from the oracle's"
    finally:
        L.free()

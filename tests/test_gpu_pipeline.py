"""GPU model pipeline (cdclq_quantize_model / cdclq_dequantize_model) on checkpoints shaped to the
reference's Hessian fixtures: byte-for-byte against the CPU restatement (tests/toy_models.py), and
the reference's own end-to-end assertions (tests/toy_models.rs): the round trip (:247-445), GPTQ and
CDCL sharing phase 1 (:452-607), act-order + skeleton through packing (:612-760); plus the error
texts of src/io.rs / src/pipeline.rs.
"""
import json
import os

import numpy as np
import pytest

import cdclq
import oracle as O
import toy_models as T

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = cdclq.Context(0)
    yield c
    c.close()


def gcfg(kw):
    return cdclq.Config(**{k: (cdclq.Method.Gptq if v == "gptq" else cdclq.Method.Cdcl) if k == "method" else v
                           for k, v in kw.items()})


def assert_same_tensors(a: dict, b: dict, label):
    assert set(a) == set(b), (label, set(a) ^ set(b))
    for k in a:
        assert a[k][0] == b[k][0] and list(a[k][1]) == list(b[k][1]), (label, k)
        assert a[k][2] == b[k][2], (label, k, "bytes differ")


@pytest.mark.parametrize("mi", range(len(T.MODELS)))
def test_pipeline_matches_the_oracle_and_the_reference_checks(ctx, tmp_path, mi):
    m = T.MODELS[mi]
    print(f"[pipeline] {m['dir']} ({m['dtype']})", flush=True)
    ck = T.make_checkpoint(m, str(tmp_path / "models" / m["dir"] / "model.safetensors"), seed=mi)
    hess = os.path.join(T.GOLDEN, m["fixture"])
    kw = T.cfg_kw(m)
    out = tmp_path / "out"
    rep = cdclq.quantize_model(ctx, [ck], [hess], out, gcfg(kw), nthreads=4)
    outs, oreps = T.oracle_quantize_model([ck], [hess], kw, nthreads=4)
    deq, _ = T.read_st(out / "dequant" / "model.safetensors")
    pk, meta = T.read_st(out / "packed" / "model.safetensors")
    assert_same_tensors(deq, outs["dequant"]["model.safetensors"], "dequant")
    assert_same_tensors(pk, outs["packed"]["model.safetensors"][0], "packed")
    assert meta == outs["packed"]["model.safetensors"][1]
    # report.json: same layers in the same order, same numbers
    assert json.load(open(out / "report.json")) == rep
    assert [l["name"] for l in rep["layers"]] == [l["name"] for l in oreps]
    for g, o in zip(rep["layers"], oreps):
        for k in ("d_out", "d_in", "subblocks_refined", "subblocks_total", "code_updates", "skeleton_groups"):
            assert g[k] == o[k], (g["name"], k)
        for k in ("loss_gptq", "loss_final", "bits_codes", "bits_total", "gain_pct"):
            assert abs(g[k] - o[k]) <= 1e-6 * max(abs(o[k]), 1e-12), (g["name"], k, g[k], o[k])
    tg = sum(l["loss_gptq"] for l in oreps)
    assert abs(rep["total_loss_gptq"] - tg) <= 1e-6 * tg
    assert rep["config"] == ("Config { bits: %d, group: %d, block: %d, damp: 0.01, act_order: true, skeleton_pct: 0.0, "
                             "skeleton_bits: 8, mse_grid: false, method: Cdcl, refine_frac: 1.0, sub_block: %d, "
                             "cd_sweeps: 1, passes: 10, tol: 0.001, refit_scales: true, row_chunk: 32 }"
                             % (kw["bits"], kw["group"], kw["block"], kw["sub_block"]))
    orig, _ = T.read_st(ck)
    T.reference_checks(m, orig, deq, pk, meta, rep["layers"], kw)
    # (7) the `cdclq dequant` path reproduces dequant/ exactly (tests/toy_models.rs:401-421)
    rt = tmp_path / "roundtrip" / "model.safetensors"
    n = cdclq.dequantize_model(ctx, out / "packed" / "model.safetensors", rt)
    assert n == len(rep["layers"])
    rts, rmeta = T.read_st(rt)
    assert rmeta == {"format": "pt"}
    assert_same_tensors(rts, deq, "roundtrip")


@pytest.mark.parametrize("mi", range(len(T.MODELS)))
def test_gptq_and_cdcl_share_phase_one(ctx, tmp_path, mi):
    """tests/toy_models.rs:452-607 on the GPU engine."""
    m = T.MODELS[mi]
    ck = T.make_checkpoint(m, str(tmp_path / "model.safetensors"), seed=10 + mi)
    tensors, _ = T.read_st(ck)
    store = T.HessStore([os.path.join(T.GOLDEN, m["fixture"])])
    base = T.cfg_kw(m)
    gptq_only = gcfg(dict(base, method="gptq", refine_frac=0.0, refit_scales=False))
    cdcl_p1 = gcfg(dict(base, method="cdcl", refine_frac=0.0, refit_scales=False))
    cdcl = gcfg(dict(base, method="cdcl", refit_scales=False))
    checked = improved = 0
    for name in sorted(tensors):
        if not name.endswith(".weight") or len(tensors[name][1]) != 2:
            continue
        layer = name[: -len(".weight")]
        owner = store.resolve(layer)
        if owner is None:
            continue
        d_out, d_in = tensors[name][1]
        w = T.decode(*tensors[name][:1], tensors[name][2], tensors[name][1])
        h = store.tensor(owner, "H")
        runs = []
        for c in (gptq_only, cdcl_p1, cdcl):
            ctx.clear_cache()
            runs.append(cdclq.quantize_layer(w, d_out, d_in, h, None, owner, c, cdclq.PrepCache(ctx=ctx), nthreads=4))
        (a, sa), (b, sb), (f, sf) = runs
        assert np.array_equal(a.perm, b.perm) and np.array_equal(a.perm, f.perm), layer
        assert np.array_equal(a.scales, b.scales) and np.array_equal(a.zeros, b.zeros), layer
        assert np.array_equal(a.codes, b.codes), layer
        assert np.array_equal(a.scales, f.scales) and np.array_equal(a.zeros, f.zeros), layer
        assert abs(sa.loss_gptq - sb.loss_gptq) <= 1e-9 * max(sa.loss_gptq, 1.0)
        assert abs(sb.loss_final - sb.loss_gptq) <= 1e-12 * max(sb.loss_gptq, 1.0)
        assert sf.loss_final <= sa.loss_gptq * (1 + 1e-9)
        # every code of the repaired layer is a legal point of its own grid
        g, ng = f.group, f.ngroups()
        gi = np.arange(d_in) // g
        maxq = ((1 << f.gbits.astype(np.int64)) - 1)[gi]
        assert (f.codes.astype(np.int64) <= maxq[None, :]).all()
        checked += 1
        if sf.loss_final < sa.loss_gptq:
            improved += 1
            assert sf.code_updates > 0
    assert checked > 0 and improved > 0


@pytest.mark.parametrize("mi", range(len(T.MODELS)))
def test_act_order_and_skeleton_survive_packing(ctx, tmp_path, mi):
    """tests/toy_models.rs:612-760: group 4, 25% skeleton, act-order; the packed perm follows the
    documented column rule; --no-dequant writes no dequant/."""
    m = T.MODELS[mi]
    ck = T.make_checkpoint(m, str(tmp_path / "model.safetensors"), seed=20 + mi)
    hess = os.path.join(T.GOLDEN, m["fixture"])
    kw = dict(T.cfg_kw(m), group=4, block=4, sub_block=2, act_order=True, skeleton_pct=25.0)
    out = tmp_path / "out"
    rep = cdclq.quantize_model(ctx, [ck], [hess], out, gcfg(kw), emit_dequant=False, nthreads=4)
    assert rep["layers"] and not (out / "dequant").exists()
    pk, _ = T.read_st(out / "packed" / "model.safetensors")
    orig, _ = T.read_st(ck)
    store = T.HessStore([hess])
    promoted = 0
    for l in rep["layers"]:
        name, d_in = l["name"], l["d_in"]
        gb = np.frombuffer(pk[f"{name}.gbits"][2], np.uint8)
        perm = np.frombuffer(pk[f"{name}.perm"][2], np.int32).astype(np.int64)
        g = int(np.frombuffer(pk[f"{name}.gsize"][2], np.int32)[0])
        if g >= d_in:
            assert (gb == kw["bits"]).all() and l["skeleton_groups"] == 0
            continue
        assert sorted(perm.tolist()) == list(range(d_in))
        ns = l["skeleton_groups"]
        assert 0 < ns < gb.size and (gb[:ns] == 8).all() and (gb[ns:] == kw["bits"]).all()
        # the documented rule: per-column saliency H_jj * ||W_:j||^2 descending (ties by index) for
        # the first ns * g columns, then the rest by descending H_jj (tests/toy_models.rs:698-741)
        h = store.tensor(store.resolve(name), "H").astype(np.float64)
        w = T.decode(orig[f"{name}.weight"][0], orig[f"{name}.weight"][2], orig[f"{name}.weight"][1])
        hd = np.diag(h).copy()
        w0 = w.astype(np.float64)
        w0[:, hd == 0.0] = 0.0
        colsq = np.zeros(d_in)
        for r in range(w0.shape[0]):  # f64 sums in row order, as the reference's loop
            colsq += w0[r] ** 2
        sal = hd * colsq
        idx = sorted(range(d_in), key=lambda j: (-sal[j], j))
        skel = idx[: ns * g]
        rest = sorted(set(range(d_in)) - set(skel), key=lambda j: (-hd[j], j))
        assert perm.tolist() == skel + rest, name
        assert perm.tolist() != list(range(d_in))
        promoted += 1
    assert promoted > 0


def test_filters_shards_and_asymmetric_hessians(ctx, tmp_path):
    """--only / --skip, two shards, an alias to a missing owner, and an M tensor (asymmetric target)
    in a second Hessian file that overrides the first one's layer."""
    m = T.MODELS[0]
    ck = T.make_checkpoint(m, str(tmp_path / "a" / "model-00001.safetensors"), seed=31)
    t, meta = T.read_st(ck)
    t2 = {k: v for k, v in t.items() if k.startswith("model.layers.1.")}
    t1 = {k: v for k, v in t.items() if not k.startswith("model.layers.1.")}
    s1, s2 = str(tmp_path / "a" / "model-00001.safetensors"), str(tmp_path / "a" / "model-00002.safetensors")
    T.write_st(s1, t1, meta)
    T.write_st(s2, t2, meta)
    hess = os.path.join(T.GOLDEN, m["fixture"])
    # override: layer 1's gate_proj gets its own H and an M (cross-covariance) in a second file
    ht, _ = T.read_st(hess)
    hh = T.decode(*ht["model.layers.1.mlp.gate_proj.H"][:1], ht["model.layers.1.mlp.gate_proj.H"][2],
                  ht["model.layers.1.mlp.gate_proj.H"][1])
    mm = (hh * np.float32(0.9)).astype(np.float32)
    h2 = str(tmp_path / "h2.safetensors")
    T.write_st(h2, {"model.layers.1.mlp.gate_proj.H": ("F32", list(hh.shape), hh.tobytes()),
                    "model.layers.1.mlp.gate_proj.M": ("F32", list(mm.shape), mm.tobytes())},
               {"aliases": json.dumps({"model.layers.1.mlp.up_proj": "model.layers.1.mlp.gate_proj",
                                       "model.layers.0.self_attn.v_proj": "does.not.exist"})})
    kw = T.cfg_kw(m)
    out = tmp_path / "out"
    only, skip = ["mlp", "v_proj"], ["down_proj"]
    rep = cdclq.quantize_model(ctx, [s1, s2], [hess, h2], out, gcfg(kw), only=only, skip=skip, nthreads=4)
    outs, oreps = T.oracle_quantize_model([s1, s2], [hess, h2], kw, only=only, skip=skip, nthreads=4)
    assert [l["name"] for l in rep["layers"]] == [l["name"] for l in oreps]
    names = [l["name"] for l in rep["layers"]]
    assert not any("down_proj" in x for x in names) and "model.layers.0.self_attn.v_proj" not in names
    assert "model.layers.1.mlp.gate_proj" in names
    for f in ("model-00001.safetensors", "model-00002.safetensors"):
        deq, _ = T.read_st(out / "dequant" / f)
        pk, pmeta = T.read_st(out / "packed" / f)
        assert_same_tensors(deq, outs["dequant"][f], f)
        assert_same_tensors(pk, outs["packed"][f][0], f)
        assert pmeta == outs["packed"][f][1]
    for g, o in zip(rep["layers"], oreps):
        assert abs(g["loss_final"] - o["loss_final"]) <= 1e-6 * o["loss_final"]


def test_error_texts(ctx, tmp_path):
    """src/io.rs:190-213 and src/pipeline.rs:137-139."""
    m = T.MODELS[0]
    ck = T.make_checkpoint(m, str(tmp_path / "model.safetensors"), seed=41)
    hess = os.path.join(T.GOLDEN, m["fixture"])
    ht, hmeta = T.read_st(hess)
    kw = T.cfg_kw(m)
    key = "model.layers.0.mlp.down_proj.H"
    h = T.decode(ht[key][0], ht[key][2], ht[key][1]).copy()
    h[3, 5] = np.nan
    bad = dict(ht)
    bad[key] = ("F32", list(h.shape), h.tobytes())
    p = str(tmp_path / "bad.safetensors")
    T.write_st(p, bad, hmeta)
    with pytest.raises(cdclq.CdclqError) as e:
        cdclq.quantize_model(ctx, [ck], [p], tmp_path / "o1", gcfg(kw))
    assert str(e.value) == (f"{key}: 64 x 64 matrix has a non-finite entry (NaN) at [ 3, 5 ]; the calibration data or "
                            "the captured forward is corrupt, refusing to quantize")
    bad[key] = ("F32", [64, 32], h[:, :32].copy().tobytes())
    T.write_st(p, bad, hmeta)
    with pytest.raises(cdclq.CdclqError) as e:
        cdclq.quantize_model(ctx, [ck], [p], tmp_path / "o2", gcfg(kw))
    assert str(e.value) == f"{key}: expected a square matrix, got [64, 32]"
    small = h[:32, :32].copy()
    small[3, 5] = 1.0
    bad[key] = ("F32", [32, 32], (small @ small.T).astype(np.float32).tobytes())
    T.write_st(p, bad, hmeta)
    with pytest.raises(cdclq.CdclqError) as e:
        cdclq.quantize_model(ctx, [ck], [p], tmp_path / "o3", gcfg(kw))
    assert str(e.value) == "model.layers.0.mlp.down_proj: Hessian is 32x32 but the weight has 64 input columns"
    # no Hessian matches: nothing quantized, everything passed through
    rep = cdclq.quantize_model(ctx, [ck], [hess], tmp_path / "o4", gcfg(kw), only=["no-such-layer"])
    assert rep["layers"] == [] and rep["total_gain_pct"] == 0.0
    orig, _ = T.read_st(ck)
    deq, _ = T.read_st(tmp_path / "o4" / "dequant" / "model.safetensors")
    assert_same_tensors(deq, orig, "pass-through")


@pytest.mark.parametrize("shape", [[2 ** 62, 4], [2 ** 62, 1], [2 ** 32, 2 ** 32, 3]])
def test_header_shape_overflow_is_rejected(ctx, tmp_path, shape):
    """A header whose element count (or byte count) wraps around 2^64 is refused with the
    safetensors crate's ValidationOverflow (checked multiplies) instead of passing the size check
    with a wrapped product of 0."""
    hdr = json.dumps({"x.weight": {"dtype": "F32", "shape": shape, "data_offsets": [0, 0]}}).encode()
    hdr += b" " * (-len(hdr) % 8)
    p = tmp_path / "overflow.safetensors"
    p.write_bytes(len(hdr).to_bytes(8, "little") + hdr)
    m = T.MODELS[0]
    hess = os.path.join(T.GOLDEN, m["fixture"])
    with pytest.raises(cdclq.CdclqError) as e:
        cdclq.quantize_model(ctx, [str(p)], [hess], tmp_path / "o", gcfg(T.cfg_kw(m)))
    assert str(e.value).endswith(": ValidationOverflow"), str(e.value)

"""GPU calibration capture (scripts/capture_hessians.py on the engine): the weighted accumulation
bit-exact against the oracle's gram on the same scaled tokens, and cdclq.capture on a small
config-built LlamaForCausalLM (random weights, no download) against a float64 torch restatement of
the reference's hooks (f32-rounding tolerance), including the alias graph, the header, split
passes, token weights, the asymmetric M, and the captured file feeding the model pipeline.
"""
import copy
import json
import os

import numpy as np
import pytest

import cdclq
import oracle as O

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ctx():
    c = cdclq.Context(0)
    yield c
    c.close()


def test_accumulate_matches_the_oracle_gram(ctx):
    rng = np.random.default_rng(3)
    t, n = 3000, 96
    x = rng.standard_normal((t, n)).astype(np.float32)
    y = (x + 0.1 * rng.standard_normal((t, n))).astype(np.float32)
    w = rng.uniform(0.2, 3.0, t).astype(np.float32)
    sw = np.sqrt(w)
    L = cdclq.lib()
    dx, dy, dw = (cdclq.DeviceArray.from_host(ctx, a) for a in (x, y, w))
    for other, label in ((None, "H"), (dy, "M")):
        acc = cdclq.DeviceArray.from_host(ctx, np.zeros((n, n)))
        for wp in (None, dw):
            acc.zero()
            yy = dx if other is None else other
            ctx.check(L.cdclq_hessian_accumulate_device(ctx.ptr, dx.ptr, yy.ptr, wp.ptr if wp is not None else None, t,
                                                        n, acc.ptr))
            xs = x if wp is None else (x * sw[:, None]).astype(np.float32)
            ys_ = (y if other is not None else x)
            ys = ys_ if wp is None else (ys_ * sw[:, None]).astype(np.float32)
            ref = O.gram_accumulate(xs, None if other is None else ys)
            got = acc.download()
            assert np.array_equal(got.view(np.uint64), ref.view(np.uint64)), label
            h = cdclq.DeviceArray(ctx, (n, n), np.float32)
            ctx.check(L.cdclq_hessian_finalize_device(ctx.ptr, acc.ptr, n, t, h.ptr))
            assert np.array_equal(h.download().view(np.uint32), (ref / t).astype(np.float32).view(np.uint32))
            h.free()
        acc.free()
    for a in (dx, dy, dw):
        a.free()


def tiny_llama(seed=0):
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(seed)
    cfg = LlamaConfig(hidden_size=64, intermediate_size=96, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, vocab_size=128, max_position_embeddings=128)
    return LlamaForCausalLM(cfg).float().to("cuda:0").eval()


def torch_reference(model, samples, batch, token_weight=None, q_model=None, skip=("lm_head",)):
    """float64 restatement of the reference's hooks (scripts/capture_hessians.py:233-245, :266)."""
    owners, probe = [], {}
    mods = [(n, m) for n, m in model.named_modules() if isinstance(m, torch.nn.Linear)
            and not any(s in n for s in skip)]
    last = {"x": None, "o": None}

    def ph(name):
        def hook(mod, inp):
            if inp[0] is last["x"]:
                probe[name] = last["o"]
                return
            last["x"], last["o"] = inp[0], name
        return hook

    hs = [m.register_forward_pre_hook(ph(n)) for n, m in mods]
    with torch.no_grad():
        model(input_ids=samples[0:1].cuda(), use_cache=False)
    for h in hs:
        h.remove()
    owners = [n for n, _ in mods if n not in probe]
    H, M, N, stash, st = {}, {}, {}, {}, {"w": None}

    def hk(name, role):
        def hook(mod, inp):
            xf = inp[0].reshape(-1, inp[0].shape[-1]).double()
            if st["w"] is not None:
                xf = xf * st["w"].double().sqrt().unsqueeze(1)
            if role == "fp" and q_model is not None:
                stash[name] = xf
                return
            H[name] = H.get(name, 0) + xf.t() @ xf
            if q_model is not None:
                M[name] = M.get(name, 0) + stash.pop(name).t() @ xf
            N[name] = N.get(name, 0) + xf.shape[0]
        return hook

    qm = dict(q_model.named_modules()) if q_model is not None else None
    hs = [dict(mods)[n].register_forward_pre_hook(hk(n, "fp")) for n in owners]
    if q_model is not None:
        hs += [qm[n].register_forward_pre_hook(hk(n, "q")) for n in owners]
    with torch.no_grad():
        for s in range(0, samples.shape[0], batch):
            ids = samples[s:s + batch].cuda()
            st["w"] = token_weight[ids].reshape(-1) if token_weight is not None else None
            model(input_ids=ids, use_cache=False)
            if q_model is not None:
                q_model(input_ids=ids, use_cache=False)
    for h in hs:
        h.remove()
    out = {f"{n}.H": (H[n] / N[n]).cpu().numpy() for n in H}
    out.update({f"{n}.M": (M[n] / N[n]).cpu().numpy() for n in M})
    return out, probe


def read(path):
    from safetensors import safe_open
    with safe_open(path, "np") as f:
        return {k: f.get_tensor(k) for k in f.keys()}, f.metadata()


def close(got, ref, label):
    scale = np.abs(ref).max()
    err = np.abs(got.astype(np.float64) - ref).max()
    assert err <= 1e-6 * scale, (label, err, scale)


def test_capture_matches_a_float64_restatement(ctx, tmp_path):
    from cdclq.capture import capture_hessians
    model = tiny_llama()
    samples = torch.randint(0, 128, (6, 48), generator=torch.Generator().manual_seed(1))
    print("[capture] tiny llama, symmetric", flush=True)
    files = capture_hessians(model, samples, str(tmp_path / "hess.safetensors"), ctx=ctx, batch=2)
    assert files == [str(tmp_path / "hess.safetensors")]
    got, meta = read(files[0])
    ref, probe = torch_reference(model, samples, 2)
    assert set(got) == set(ref)
    for k in ref:
        close(got[k], ref[k], k)
    assert meta["format"] == "hessian_v1" and meta["generator"] == "cdclq-capture"
    assert meta["calib_tokens"] == str(6 * 48)
    aliases = json.loads(meta["aliases"])
    assert aliases == probe
    for i in range(2):
        p = f"model.layers.{i}."
        assert aliases[p + "self_attn.k_proj"] == p + "self_attn.q_proj"
        assert aliases[p + "self_attn.v_proj"] == p + "self_attn.q_proj"
        assert aliases[p + "mlp.up_proj"] == p + "mlp.gate_proj"


def test_split_passes_equal_one_pass(ctx, tmp_path):
    """scripts/capture_hessians.py:40-45: a split Hessian is bit-identical to a single-pass one."""
    from cdclq.capture import capture_hessians, plan_entry_bytes
    model = tiny_llama(1)
    samples = torch.randint(0, 128, (4, 40), generator=torch.Generator().manual_seed(2))
    one = capture_hessians(model, samples, str(tmp_path / "one.safetensors"), ctx=ctx, batch=2)
    budget = (plan_entry_bytes(96) + plan_entry_bytes(64)) / (1 << 30)
    many = capture_hessians(model, samples, str(tmp_path / "split.safetensors"), ctx=ctx, batch=2,
                            max_hessian_mem=budget)
    assert len(many) > 1 and all(".of" not in p and "of" in os.path.basename(p) for p in many)
    t1, m1 = read(one[0])
    merged, aliases = {}, {}
    for p in many:
        t, m = read(p)
        merged.update(t)
        aliases.update(json.loads(m["aliases"]))
    assert set(merged) == set(t1) and aliases == json.loads(m1["aliases"])
    for k in t1:
        assert np.array_equal(merged[k].view(np.uint32), t1[k].view(np.uint32)), k


def test_token_weights_and_asymmetric_m(ctx, tmp_path):
    from cdclq.capture import capture_hessians
    model = tiny_llama(2)
    q_model = copy.deepcopy(model)
    with torch.no_grad():  # perturb the first layer so the later layers' inputs differ (x~ != x)
        for p in q_model.model.layers[0].parameters():
            p.add_(0.01 * torch.randn_like(p))
    samples = torch.randint(0, 128, (4, 32), generator=torch.Generator().manual_seed(3))
    tw = torch.ones(128, device="cuda:0")
    tw[::7] = 3.0
    files = capture_hessians(model, samples, str(tmp_path / "hm.safetensors"), ctx=ctx, batch=2, token_weight=tw,
                             q_model=q_model)
    got, _ = read(files[0])
    ref, _ = torch_reference(model, samples, 2, token_weight=tw, q_model=q_model)
    assert set(got) == set(ref) and any(k.endswith(".M") for k in got)
    for k in ref:
        close(got[k], ref[k], k)
    k = "model.layers.1.self_attn.q_proj"
    assert not np.allclose(got[k + ".M"], got[k + ".H"])  # the perturbation reached layer 1


def test_captured_hessians_feed_the_pipeline(ctx, tmp_path):
    """capture -> quantize_model: every Linear but lm_head is quantized through the aliases."""
    from cdclq.capture import capture_hessians
    from safetensors.torch import save_file
    model = tiny_llama(4)
    samples = torch.randint(0, 128, (8, 64), generator=torch.Generator().manual_seed(5))
    hess = capture_hessians(model, samples, str(tmp_path / "hess.safetensors"), ctx=ctx, batch=4)
    ck = str(tmp_path / "model" / "model.safetensors")
    os.makedirs(os.path.dirname(ck))
    save_file({k: v.detach().to(torch.bfloat16).cpu().contiguous() for k, v in model.state_dict().items()}, ck)
    rep = cdclq.quantize_model(ctx, [ck], hess, tmp_path / "out", cdclq.Config(bits=4, group=32, block=32), nthreads=4)
    names = {l["name"] for l in rep["layers"]}
    lin = {n for n, m in model.named_modules() if isinstance(m, torch.nn.Linear) and n != "lm_head"}
    assert names == lin
    assert rep["total_loss_final"] <= rep["total_loss_gptq"]

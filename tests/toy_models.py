"""Toy checkpoints and a CPU restatement of the model pipeline, for the end-to-end tests.

TEST INFRASTRUCTURE. The reference's end-to-end suite (tests/toy_models.rs) runs three tiny
Llama-family checkpoints against its committed Hessian fixtures; the checkpoints themselves are
downloaded there and are not part of /root/reference. Here the checkpoints are synthetic: the same
tensor names, the Llama layout and storage dtypes (f16 / bf16 / f32), with every `.weight` shaped to
the committed Hessians (tests/golden/hess_*.safetensors, the reference's fixtures) and random values.

`oracle_quantize_model` restates pipeline::quantize_model (src/pipeline.rs:79-227) on the CPU
oracle: the same job selection and order, the same PrepCache per shard, the dequant/ tensors in the
checkpoint dtype and the six packed tensors, as {file: {name: (dtype, shape, bytes)}}.
"""
from __future__ import annotations

import json
import os
import struct

import numpy as np

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# tests/toy_models.rs:43-58 (model settings), with the synthetic checkpoint shapes
MODELS = [
    dict(dir="tiny-random-Llama-3", fixture="hess_tiny-random-Llama-3.safetensors", dtype="F16", bits=4, group=16,
         block=16, q_out=16, kv_out=8),
    dict(dir="llama-3", fixture="hess_llama-3.safetensors", dtype="BF16", bits=3, group=8, block=8, q_out=512,
         kv_out=64),
    dict(dir="tiny-random-llama2", fixture="hess_tiny-random-llama2.safetensors", dtype="F32", bits=3, group=32,
         block=32, q_out=256, kv_out=128),
]

DSIZE = {"F32": 4, "F16": 2, "BF16": 2, "U8": 1, "I32": 4, "F64": 8, "I64": 8, "U16": 2, "I16": 2, "U32": 4, "I8": 1,
         "BOOL": 1, "U64": 8}


def cfg_kw(m: dict) -> dict:
    """tests/toy_models.rs:88-98"""
    return dict(bits=m["bits"], group=m["group"], block=m["block"], sub_block=max(m["block"] // 2, 1), damp=0.01,
                row_chunk=32)


# ---------------------------------------------------------------- raw safetensors (header + bytes)
def read_st(path):
    """{name: (dtype, shape, bytes)}, metadata"""
    b = open(path, "rb").read()
    n = struct.unpack("<Q", b[:8])[0]
    h = json.loads(b[8:8 + n])
    meta = h.pop("__metadata__", {}) or {}
    base = 8 + n
    out = {}
    for k, v in h.items():
        a, e = v["data_offsets"]
        out[k] = (v["dtype"], list(v["shape"]), b[base + a:base + e])
    return out, meta


def write_st(path, tensors: dict, meta: dict | None = None):
    """tensors: {name: (dtype, shape, bytes)}"""
    os.makedirs(os.path.dirname(path) or ".", exist_ok=True)
    hdr = {}
    if meta:
        hdr["__metadata__"] = meta
    off = 0
    blobs = []
    for k in sorted(tensors):
        dt, sh, by = tensors[k]
        hdr[k] = {"dtype": dt, "shape": list(sh), "data_offsets": [off, off + len(by)]}
        off += len(by)
        blobs.append(by)
    hj = json.dumps(hdr, separators=(",", ":")).encode()
    hj += b" " * ((8 - len(hj) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for by in blobs:
            f.write(by)


def decode(dtype: str, raw: bytes, shape) -> np.ndarray:
    """io::tensor_to_f32 (src/io.rs:37-45), finite inputs."""
    if dtype == "F32":
        return np.frombuffer(raw, np.float32).reshape(shape).copy()
    if dtype == "F16":
        return np.frombuffer(raw, np.float16).astype(np.float32).reshape(shape)
    if dtype == "BF16":
        return (np.frombuffer(raw, np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(shape)
    raise ValueError(f"unsupported weight dtype {dtype} (need F32/F16/BF16)")


def encode(dtype: str, v: np.ndarray) -> bytes:
    return O.narrow(np.ascontiguousarray(v, np.float32), dtype).tobytes()


# ---------------------------------------------------------------- synthetic checkpoints
def hessian_layers(fixture_path):
    t, meta = read_st(fixture_path)
    owners = {k[:-2]: v[1][0] for k, v in t.items() if k.endswith(".H")}
    aliases = json.loads(meta.get("aliases", "{}"))
    return owners, aliases


def make_checkpoint(m: dict, path: str, seed: int = 0):
    """A Llama-layout checkpoint whose `.weight` shapes match the model's Hessian fixture; also the
    uncalibrated tensors the pipeline must pass through (embeddings, lm_head, norms)."""
    owners, aliases = hessian_layers(os.path.join(GOLDEN, m["fixture"]))
    rng = np.random.default_rng(seed)
    layers = sorted({k.rsplit(".", 2)[0] for k in list(owners) + list(aliases)})  # "model.layers.<i>"
    hidden = [v for k, v in owners.items() if k.endswith("self_attn.k_proj")][0]
    inter = [v for k, v in owners.items() if k.endswith("mlp.down_proj")][0]
    dt = m["dtype"]
    tensors = {}

    def put(name, shape, scale=0.02):
        v = (rng.standard_normal(shape) * scale).astype(np.float32)
        tensors[name] = (dt, list(shape), encode(dt, v))

    for pre in layers:
        for proj in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
                     "mlp.up_proj", "mlp.down_proj"):
            layer = f"{pre}.{proj}"
            own = layer if layer in owners else aliases.get(layer)
            d_in = owners[own] if own in owners else (inter if proj.endswith("down_proj") else hidden)
            d_out = {"q_proj": m["q_out"], "k_proj": m["kv_out"], "v_proj": m["kv_out"], "o_proj": hidden,
                     "gate_proj": inter, "up_proj": inter, "down_proj": hidden}[proj.split(".")[1]]
            put(layer + ".weight", (d_out, d_in))
        put(pre + ".input_layernorm.weight", (hidden,), 1.0)
        put(pre + ".post_attention_layernorm.weight", (hidden,), 1.0)
    put("model.embed_tokens.weight", (32, hidden))
    put("lm_head.weight", (32, hidden))
    put("model.norm.weight", (hidden,), 1.0)
    write_st(path, tensors, {"format": "pt"})
    return path


# ---------------------------------------------------------------- CPU pipeline
class HessStore:
    """io::HessianStore (src/io.rs:150-226)"""

    def __init__(self, paths):
        self.files, self.index, self.aliases = [], {}, {}
        for fi, p in enumerate(paths):
            t, meta = read_st(p)
            self.files.append(t)
            for k in t:
                if k.endswith(".H"):
                    self.index[k[:-2]] = fi
            if "aliases" in meta:
                self.aliases.update(json.loads(meta["aliases"]))

    def resolve(self, layer):
        if layer in self.index:
            return layer
        o = self.aliases.get(layer)
        return o if o in self.index else None

    def tensor(self, owner, suffix):
        t = self.files[self.index[owner]]
        key = f"{owner}.{suffix}"
        if key not in t:
            return None
        dt, sh, raw = t[key]
        assert len(sh) == 2 and sh[0] == sh[1], key
        v = decode(dt, raw, sh)
        assert np.isfinite(v).all(), key
        return v


def oracle_quantize_model(weights, hessians, cfg: dict, only=(), skip=(), emit_packed=True, emit_dequant=True,
                          nthreads=1):
    """pipeline::quantize_model (src/pipeline.rs:79-227) on the CPU oracle:
    ({"dequant": {file: tensors}, "packed": {file: (tensors, meta)}}, [layer report dicts])."""
    store = HessStore(hessians)
    ocfg = O.config(**cfg)
    outs = {"dequant": {}, "packed": {}}
    reports = []
    for shard in weights:
        tensors, _ = read_st(shard)
        names = sorted(tensors)
        jobs = []
        for name in names:
            if not name.endswith(".weight"):
                continue
            layer = name[: -len(".weight")]
            if len(tensors[name][1]) != 2:
                continue
            if only and not any(s in layer for s in only):
                continue
            if any(s in layer for s in skip):
                continue
            owner = store.resolve(layer)
            if owner is not None:
                jobs.append((name, layer, owner))
        jobs.sort(key=lambda j: (j[2], j[1]))
        cache = O.Cache()
        deq, pk, done, orig = {}, {}, set(), None
        for name, layer, owner in jobs:
            dt, sh, raw = tensors[name]
            w = decode(dt, raw, sh)
            h = store.tensor(owner, "H")
            assert h.shape[0] == sh[1]
            mm = store.tensor(owner, "M")
            q = O.quantize_layer(w, h, ocfg, m=mm, hkey=owner, cache=cache, nthreads=nthreads)
            s = q.stats
            gain = 100.0 * (s["loss_gptq"] - s["loss_final"]) / s["loss_gptq"] if s["loss_gptq"] > 0 else 0.0
            reports.append(dict(name=layer, d_out=sh[0], d_in=sh[1], gain_pct=gain, **{k: s[k] for k in (
                "loss_gptq", "loss_final", "subblocks_refined", "subblocks_total", "code_updates", "skeleton_groups",
                "bits_codes", "bits_total")}))
            orig = orig or dt
            if emit_dequant:
                deq[name] = (dt, list(sh), O.narrow(q.dequantize(), dt).tobytes())
            if emit_packed:
                qw, s16, qz, p32 = O.pack_layer(q.codes, q.scales, q.zeros, q.perm, q.gbits, q.group)
                ng = q.gbits.size
                pk[f"{layer}.qweight"] = ("U8", [sh[0], qw.shape[1]], qw.tobytes())
                pk[f"{layer}.scales"] = ("F16", [sh[0], ng], s16.tobytes())
                pk[f"{layer}.qzeros"] = ("U8", [sh[0], ng], qz.tobytes())
                pk[f"{layer}.perm"] = ("I32", [sh[1]], p32.tobytes())
                pk[f"{layer}.gbits"] = ("U8", [ng], q.gbits.tobytes())
                pk[f"{layer}.gsize"] = ("I32", [1], np.array([q.group], np.int32).tobytes())
            done.add(name)
        for name in names:
            if name in done:
                continue
            if emit_dequant:
                deq[name] = tensors[name]
            if emit_packed:
                pk[name] = tensors[name]
        fname = os.path.basename(shard)
        if emit_dequant and deq:
            outs["dequant"][fname] = deq
        if emit_packed and pk:
            meta = {"format": "pt", "quantization": "cdclq-v1", "orig_dtype": orig or "F16", "bits": str(cfg["bits"])}
            outs["packed"][fname] = (pk, meta)
    return outs, reports


# ---------------------------------------------------------------- tests/toy_models.rs:247-445 checks
def damped_permuted_h(h, perm, damp):
    """tests/toy_models.rs:199-222"""
    n = h.shape[0]
    hp = h.astype(np.float64)[np.ix_(perm, perm)]
    d = np.diag(hp).copy()
    d[d == 0.0] = 1.0
    np.fill_diagonal(hp, d)
    hp[np.diag_indices(n)] += damp * d.mean()
    return hp.astype(np.float32)


def reference_checks(m, orig, deq, pk, pk_meta, reports, cfg):
    """The assertions of toy_checkpoint_quantize_and_roundtrip (tests/toy_models.rs:247-445), (1)-(6)
    and (8), on one model's outputs ({name: (dtype, shape, bytes)} dicts)."""
    assert reports, "no layer quantized"
    # (1) same tensor set, shapes and dtypes
    assert set(orig) == set(deq)
    for k in orig:
        assert orig[k][:2] == deq[k][:2], k
    store = HessStore([os.path.join(GOLDEN, m["fixture"])])
    for l in reports:
        name = l["name"]
        # (2) six companion tensors; the reader path reproduces dequant/ exactly
        for suf in ("qweight", "scales", "qzeros", "perm", "gbits", "gsize"):
            assert f"{name}.{suf}" in pk, (name, suf)
        qw = np.frombuffer(pk[f"{name}.qweight"][2], np.uint8).reshape(pk[f"{name}.qweight"][1])
        s16 = np.frombuffer(pk[f"{name}.scales"][2], np.uint16)
        qz = np.frombuffer(pk[f"{name}.qzeros"][2], np.uint8)
        p32 = np.frombuffer(pk[f"{name}.perm"][2], np.int32)
        gb = np.frombuffer(pk[f"{name}.gbits"][2], np.uint8)
        g = int(np.frombuffer(pk[f"{name}.gsize"][2], np.int32)[0])
        d_out, d_in = qw.shape[0], p32.size
        assert (d_out, d_in) == (l["d_out"], l["d_in"])
        dt = deq[f"{name}.weight"][0]
        assert O.dequantize_packed(qw, s16, qz, p32, gb, g, dt).tobytes() == deq[f"{name}.weight"][2], name
        # (3) every code fits its group's width
        codes = np.stack([O.unpack_row(qw[r], d_in, g, gb) for r in range(d_out)])
        widths = gb.astype(np.int64)[np.arange(d_in) // g]
        assert (codes.astype(np.int64) < (1 << widths)).all(), name
        # (4) the reported loss from the packed file alone, H damped and permuted independently
        hv = store.tensor(store.resolve(name), "H")
        w = decode(*orig[f"{name}.weight"][:1], orig[f"{name}.weight"][2], orig[f"{name}.weight"][1])
        w0 = w.copy()
        w0[:, np.diag(hv) == 0.0] = 0.0
        perm = p32.astype(np.int64)
        hd = damped_permuted_h(hv, perm, cfg["damp"]).astype(np.float64)
        ng = gb.size
        sc = s16.view(np.float16).astype(np.float32).reshape(d_out, ng)[:, np.arange(d_in) // g]
        zr = qz.astype(np.float32).reshape(d_out, ng)[:, np.arange(d_in) // g]
        e = (w0[:, perm] - sc * (codes.astype(np.float32) - zr)).astype(np.float64)
        loss = float(np.einsum("ij,jk,ik->", e, hd, e))
        assert loss > 0 and abs(loss - l["loss_final"]) / loss <= 5e-3, (name, loss, l["loss_final"])
        assert l["loss_final"] <= l["loss_gptq"] * (1 + 1e-9), name
    # (5) exact pass-through
    quantized = {f"{l['name']}.weight" for l in reports}
    untouched = [k for k in orig if k not in quantized]
    for k in untouched:
        assert orig[k] == deq[k], k
    assert len(untouched) >= 2
    # (6) the packed header
    assert pk_meta.get("quantization") == "cdclq-v1" and "orig_dtype" in pk_meta
    # (8) packed codes are much smaller than the weights they replace
    orig_bytes = sum(len(orig[k][2]) for k in quantized)
    qw_bytes = sum(len(v[2]) for k, v in pk.items() if k.endswith(".qweight"))
    assert qw_bytes * 2 < orig_bytes

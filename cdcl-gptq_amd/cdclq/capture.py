"""Calibration capture on the GPU engine: scripts/capture_hessians.py of the reference, with the
`addmm_` accumulation replaced by cdclq_hessian_accumulate_device.

For every matched nn.Linear of a (PyTorch-ROCm) model it accumulates

    H = (1/N) * sum_t  w_t * x_t x_t^T          (scripts/capture_hessians.py:233-245, :266)

over the calibration tokens (x_t = the layer input at token t, w_t = optional per-token weight),
and writes `<module>.H` (float32) to safetensors with the reference's header (`format: hessian_v1`,
`generator`, `calib_tokens`, `aliases`). Modules that receive the very same input tensor (q/k/v,
gate/up) are found by a probe forward pass (tensor identity, :185-208) and stored once, the later
ones recorded in `aliases`. `max_hessian_mem` bounds the accumulators; above it the distinct inputs
are packed into bins (first-fit decreasing, largest first, :73-101) and captured in one forward
pass per bin, one file per bin (`<stem>.<i>of<n>.safetensors`).

Differences from the reference, by design:
  * accumulation: each batch's tokens are summed as f32 fused-multiply-add chains over 2048-token
    chunks, chunks in f64 (the engine's gram_accumulate), then divided by N in f64 and rounded once
    to f32. The reference accumulates in f32 through torch.addmm in an unspecified order, so the
    two agree to f32 rounding, not bit for bit. The accumulators are f64 (8 bytes per entry), and
    `max_hessian_mem` budgets them as such.
  * asymmetric calibration: given `q_model` (the same architecture with quantized inputs upstream),
    each owner also gets `<module>.M` = (1/N) sum_t w_t x_t x~_t^T (x from `model`, x~ from
    `q_model` at the same tokens) and `.H` becomes the x~ Hessian, the pair the engine's asymmetric
    target takes (src/engine.rs:690-699). The reference's capture writes H only.

Device pointers of torch tensors are handed to the library after a synchronisation of torch's
current stream; every library call returns after its device work finished.
"""
from __future__ import annotations

import json
import os
import sys

from . import CdclqError, Context, lib

GIB = 1 << 30


def accumulator_bytes(d_in: int) -> int:
    """One f64 d_in x d_in accumulator."""
    return d_in * d_in * 8


def fmt_bytes(n: int) -> str:
    """scripts/capture_hessians.py:63-70"""
    if n >= GIB:
        return f"{n / GIB:.2f} GiB"
    if n >= 1 << 20:
        return f"{n / (1 << 20):.1f} MiB"
    return f"{n / (1 << 10):.1f} KiB"


def plan_bins(families: dict, budget: int) -> list:
    """scripts/capture_hessians.py:73-101: pack owner inputs (name -> d_in) into bins of at most
    `budget` bytes, first-fit decreasing, largest family first (ties by name)."""
    bins: list = []
    for owner, d_in in sorted(families.items(), key=lambda kv: (-accumulator_bytes(kv[1]), kv[0])):
        need = accumulator_bytes(d_in)
        if need > budget:
            raise ValueError(
                f"{owner}: a single Hessian at d_in={d_in} is {fmt_bytes(need)}, above the budget "
                f"{fmt_bytes(budget)}. Raise the budget, or capture this layer in its own run with only=[...].")
        for b in bins:
            if b["bytes"] + need <= budget:
                b["bytes"] += need
                b["owners"].append(owner)
                break
        else:
            bins.append({"bytes": need, "owners": [owner]})
    return bins


def out_path_for(out: str, i: int, n: int) -> str:
    """scripts/capture_hessians.py:104-110"""
    if n == 1:
        return out
    stem, ext = os.path.splitext(out)
    return f"{stem}.{i}of{n}{ext}"


def _check(ctx: Context, rc: int):
    if rc != 0:
        raise CdclqError(rc, lib().cdclq_last_error(ctx.ptr).decode())


def capture_hessians(model, samples, out: str, ctx: Context | None = None, batch: int = 2, token_weight=None,
                     only=(), skip=("lm_head",), max_hessian_mem: float = 64.0, q_model=None, log=sys.stderr):
    """Capture the Hessians of `model` (on the GPU of `ctx`) over `samples` (nsamples x seqlen token
    ids), scripts/capture_hessians.py:112-330. token_weight: optional per-vocabulary-entry weight
    (a float tensor indexed by token id, the reference's `--struct-weight` table). Returns the list
    of files written."""
    import torch
    import torch.nn as nn

    ctx = ctx or Context(0)
    dev = next(model.parameters()).device
    targets = []
    for name, mod in model.named_modules():
        if not isinstance(mod, nn.Linear):
            continue
        if only and not any(s in name for s in only):
            continue
        if any(s in name for s in skip):
            continue
        targets.append((name, mod))
    if not targets:
        raise ValueError("no Linear module matched only/skip")
    qmods = dict(q_model.named_modules()) if q_model is not None else None
    nsamples = samples.shape[0]

    # probe: the sharing graph from the identity of the input tensors (:185-208)
    probe: dict = {}
    pst = {"last_x": None, "last_owner": None}

    def make_probe(name):
        def hook(module, inputs):
            x = inputs[0]
            if x is pst["last_x"]:
                probe[name] = pst["last_owner"]
                return
            pst["last_x"], pst["last_owner"] = x, name
        return hook

    hs = [mod.register_forward_pre_hook(make_probe(name)) for name, mod in targets]
    with torch.no_grad():
        model(input_ids=samples[0:1].to(dev), use_cache=False)
    for h in hs:
        h.remove()
    pst["last_x"] = None

    families = {name: mod.in_features for name, mod in targets if name not in probe}
    per_owner = 2 if q_model is not None else 1  # H and M accumulators
    bins = plan_bins(families, int(max_hessian_mem * GIB / per_owner))
    total = sum(accumulator_bytes(d) for d in families.values()) * per_owner
    print(f"{len(targets)} Linear modules, {len(families)} distinct layer inputs ({len(probe)} aliased) = "
          f"{fmt_bytes(total)} of accumulators; {len(bins)} pass(es)", file=log)

    L = lib()
    written = []
    for bi, b in enumerate(bins, 1):
        owners = set(b["owners"])
        acc, macc, count, stash = {}, {}, {}, {}
        state = {"w": None}

        def sync():
            torch.cuda.current_stream(dev).synchronize()

        def make_hook(name, role):
            def hook(module, inputs):
                x = inputs[0]
                xf = x.reshape(-1, x.shape[-1]).float().contiguous()
                w = state["w"]
                t, n = xf.shape
                if role == "fp" and q_model is not None:
                    stash[name] = xf  # paired with the quantized model's input at the same tokens
                    return
                if name not in acc:
                    acc[name] = torch.zeros(n, n, dtype=torch.float64, device=dev)
                    count[name] = 0
                    if q_model is not None:
                        macc[name] = torch.zeros(n, n, dtype=torch.float64, device=dev)
                sync()
                wp = w.data_ptr() if w is not None else None
                _check(ctx, L.cdclq_hessian_accumulate_device(ctx.ptr, xf.data_ptr(), xf.data_ptr(), wp, t, n,
                                                               acc[name].data_ptr()))
                if q_model is not None:
                    xs = stash.pop(name)
                    _check(ctx, L.cdclq_hessian_accumulate_device(ctx.ptr, xs.data_ptr(), xf.data_ptr(), wp, t, n,
                                                                   macc[name].data_ptr()))
                count[name] += t
            return hook

        handles = [mod.register_forward_pre_hook(make_hook(name, "fp")) for name, mod in targets if name in owners]
        if q_model is not None:
            handles += [qmods[name].register_forward_pre_hook(make_hook(name, "q")) for name, _ in targets
                        if name in owners]
        nb = (nsamples + batch - 1) // batch
        with torch.no_grad():
            for s in range(0, nsamples, batch):
                ids = samples[s:s + batch].to(dev)
                state["w"] = (token_weight[ids].reshape(-1).float().contiguous()
                              if token_weight is not None else None)
                model(input_ids=ids, use_cache=False)
                if q_model is not None:
                    q_model(input_ids=ids, use_cache=False)
                print(f"pass {bi}/{len(bins)} batch {s // batch + 1}/{nb}", file=log)
        for h in handles:
            h.remove()

        aliases_here = {dep: own for dep, own in probe.items() if own in owners}
        seen = set(count.values())
        meta = {"format": "hessian_v1", "generator": "cdclq-capture", "calib_tokens": str(max(seen)),
                "aliases": json.dumps(aliases_here)}
        if len(seen) > 1:
            meta["calib_tokens_min"] = str(min(seen))
        tensors = {}
        for name in acc:
            n = acc[name].shape[0]
            for suffix, a in (("H", acc[name]), ("M", macc.get(name))):
                if a is None:
                    continue
                h32 = torch.empty(n, n, dtype=torch.float32, device=dev)
                _check(ctx, L.cdclq_hessian_finalize_device(ctx.ptr, a.data_ptr(), n, count[name], h32.data_ptr()))
                tensors[f"{name}.{suffix}"] = h32.cpu().contiguous()
        path = out_path_for(out, bi, len(bins))
        os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
        from safetensors.torch import save_file
        save_file(tensors, path, metadata=meta)
        written.append(path)
        print(f"saved {len(acc)} Hessian(s) ({len(aliases_here)} aliased) -> {path}", file=log)
        del acc, macc, tensors
    return written

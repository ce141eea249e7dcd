"""Calibration capture on the GPU engine: the job of the reference's scripts/capture_hessians.py,
with its per-batch `addmm_` replaced by cdclq_hessian_accumulate_device.

For every matched nn.Linear of a (PyTorch-ROCm) model it builds

    H = (1/N) * sum_t  w_t * x_t x_t^T          (scripts/capture_hessians.py:233-245, :266)

over the calibration tokens (x_t = the layer input at token t, w_t = optional per-token weight)
and writes `<module>.H` (float32) to safetensors.

What must agree with the reference, because other tools read the files:
  * the header keys `format` = "hessian_v1", `generator`, `calib_tokens` (+ `calib_tokens_min`
    when layers saw different token counts) and `aliases` (JSON: module -> the owner whose H it
    shares);
  * the sharing graph: a module whose forward input is the very tensor object the previously
    hooked module received (q/k/v behind one norm, gate/up) stores nothing and is an alias
    (scripts/capture_hessians.py:185-208);
  * the split into passes when the accumulators exceed `max_hessian_mem`, which decides which file
    holds which Hessian: planned with the reference's weight of 4 bytes per entry
    (scripts/capture_hessians.py:59-61, :76-102), one file per pass named <stem>.<i>of<n><ext>.

What differs, by design:
  * accumulation: each batch is summed as the engine's gram_accumulate (f32 fused-multiply-add
    chains over 2048-token chunks, f64 across chunks), divided by N in f64 and rounded once to f32.
    The reference sums in f32 through torch.addmm in an order its BLAS picks, so the two agree to
    f32 rounding, not bit for bit. The device accumulators are f64 (8 bytes per entry, twice that
    with `q_model`); a pass that does not fit the GPU's free memory is refused before it starts.
  * asymmetric calibration: given `q_model` (the same architecture with quantized layers
    upstream), each owner also gets `<module>.M` = (1/N) sum_t w_t x_t x~_t^T (x from `model`, x~
    from `q_model` at the same tokens) and `.H` becomes the x~ Hessian: the pair the engine's
    asymmetric target takes (src/engine.rs:690-699). The reference's capture writes H only.

Device pointers of torch tensors are handed to the library after torch's current stream is
synchronised; every library call returns after its device work finished.
"""
from __future__ import annotations

import json
import os
import sys
from dataclasses import dataclass, field

from . import CdclqError, Context, lib

GIB = 1 << 30


def plan_entry_bytes(d_in: int) -> int:
    """What one owner weighs in the pass plan: a d_in x d_in float32 matrix, the reference's
    accounting (it accumulates in f32), so the same budget gives the same files."""
    return 4 * d_in * d_in


def device_entry_bytes(d_in: int, paired: bool) -> int:
    """Device memory one owner really takes here: an f64 accumulator, two when M is captured too."""
    return 8 * d_in * d_in * (2 if paired else 1)


def human_size(nbytes: int) -> str:
    """Bytes in the largest binary unit that keeps the number at or above 1 (KiB at least)."""
    for unit, shift, digits in (("GiB", 30, 2), ("MiB", 20, 1)):
        if nbytes >= 1 << shift:
            return f"{nbytes / (1 << shift):.{digits}f} {unit}"
    return f"{nbytes / 1024:.1f} KiB"


@dataclass
class CapturePass:
    """Owners captured in one forward sweep, and their planned bytes."""

    owners: list = field(default_factory=list)
    planned: int = 0


def plan_passes(widths: dict, budget: int) -> list:
    """Distribute the owners (name -> d_in) over capture passes of at most `budget` planned bytes.

    The plan is the reference's (scripts/capture_hessians.py:76-102), kept because it fixes which
    file receives which Hessian: owners are taken from the largest accumulator down (by name among
    equal sizes) and each goes to the earliest pass that still has room for it, or opens a new
    pass. An owner that alone exceeds the budget cannot be captured."""
    passes: list = []
    for owner in sorted(widths, key=lambda o: (-plan_entry_bytes(widths[o]), o)):
        size = plan_entry_bytes(widths[owner])
        if size > budget:
            raise ValueError(f"{owner} (d_in={widths[owner]}) needs {human_size(size)} for its Hessian alone, more "
                             f"than max_hessian_mem = {human_size(budget)}; raise the budget or capture this module "
                             f"in a run of its own (only=[...])")
        home = next((p for p in passes if p.planned + size <= budget), None)
        if home is None:
            home = CapturePass()
            passes.append(home)
        home.owners.append(owner)
        home.planned += size
    return passes


def pass_file(out: str, index: int, count: int) -> str:
    """File of pass `index` (1-based) of `count`: `out` itself when there is one pass, otherwise
    `out` with `.<index>of<count>` before its extension (the reference's file naming)."""
    if count == 1:
        return out
    root, ext = os.path.splitext(out)
    return f"{root}.{index}of{count}{ext}"


class SharedInputProbe:
    """Finds the modules that share a forward input. A hooked module that receives the same tensor
    object as the module hooked just before it is an alias of that module's owner; any other input
    starts a new family owned by the receiving module."""

    def __init__(self):
        self.alias_of: dict = {}
        self._last = None  # (input tensor, owner of its family)

    def hook(self, name: str):
        def on_input(module, inputs):
            x = inputs[0]
            if self._last is not None and x is self._last[0]:
                self.alias_of[name] = self._last[1]
            else:
                self._last = (x, name)
        return on_input

    def release(self):
        self._last = None


class _PassAccumulators:
    """Device accumulators of one capture pass: H (and M when a quantized twin is given) per owner,
    token counts, and the full-precision inputs waiting for their quantized-model partners."""

    def __init__(self, ctx: Context, device, paired: bool):
        self.ctx, self.device, self.paired = ctx, device, paired
        self.h: dict = {}
        self.m: dict = {}
        self.tokens: dict = {}
        self.pending: dict = {}
        self.weights = None  # per-token weights of the current batch (float32, device) or None

    def _call(self, rc: int):
        if rc != 0:
            raise CdclqError(rc, lib().cdclq_last_error(self.ctx.ptr).decode())

    def hook(self, name: str, source: str):
        """Forward pre-hook on `name`; source "fp" for `model`, "q" for `q_model`."""
        import torch

        def on_input(module, inputs):
            x = inputs[0]
            rows = x.reshape(-1, x.shape[-1]).float().contiguous()
            if self.paired and source == "fp":
                self.pending[name] = rows  # paired with the quantized model's input at the same tokens
                return
            t, n = rows.shape
            if name not in self.h:
                self.h[name] = torch.zeros(n, n, dtype=torch.float64, device=self.device)
                self.tokens[name] = 0
                if self.paired:
                    self.m[name] = torch.zeros(n, n, dtype=torch.float64, device=self.device)
            torch.cuda.current_stream(self.device).synchronize()
            wp = self.weights.data_ptr() if self.weights is not None else None
            L = lib()
            self._call(L.cdclq_hessian_accumulate_device(self.ctx.ptr, rows.data_ptr(), rows.data_ptr(), wp, t, n,
                                                         self.h[name].data_ptr()))
            if self.paired:
                xs = self.pending.pop(name)
                self._call(L.cdclq_hessian_accumulate_device(self.ctx.ptr, xs.data_ptr(), rows.data_ptr(), wp, t, n,
                                                             self.m[name].data_ptr()))
            self.tokens[name] += t
        return on_input

    def finalize(self) -> dict:
        """name.H / name.M -> float32 host tensors, each (1/N) * accumulator rounded once."""
        import torch

        out = {}
        for name, acc in self.h.items():
            n = acc.shape[0]
            for suffix, a in (("H", acc), ("M", self.m.get(name))):
                if a is None:
                    continue
                h32 = torch.empty(n, n, dtype=torch.float32, device=self.device)
                self._call(lib().cdclq_hessian_finalize_device(self.ctx.ptr, a.data_ptr(), n, self.tokens[name],
                                                               h32.data_ptr()))
                out[f"{name}.{suffix}"] = h32.cpu().contiguous()
        return out


def _header(tokens: dict, aliases: dict) -> dict:
    """The reference's safetensors metadata (hessian_v1)."""
    counts = sorted(set(tokens.values()))
    meta = {"format": "hessian_v1", "generator": "cdclq-capture", "calib_tokens": str(counts[-1]),
            "aliases": json.dumps(aliases)}
    if len(counts) > 1:
        meta["calib_tokens_min"] = str(counts[0])
    return meta


def capture_hessians(model, samples, out: str, ctx: Context | None = None, batch: int = 2, token_weight=None,
                     only=(), skip=("lm_head",), max_hessian_mem: float = 6.0, q_model=None, log=sys.stderr):
    """Capture the Hessians of `model` (on the GPU of `ctx`) over `samples` (nsamples x seqlen
    token ids): the job of scripts/capture_hessians.py:112-330. token_weight: optional weight per
    vocabulary entry (a float tensor indexed by token id, the reference's --struct-weight table).
    max_hessian_mem: GiB of planned accumulators per pass (the reference's --max-hessian-mem,
    default 6). Returns the files written, one per pass."""
    import torch
    import torch.nn as nn

    ctx = ctx or Context(0)
    dev = next(model.parameters()).device

    def wanted(name: str) -> bool:
        return (not only or any(s in name for s in only)) and not any(s in name for s in skip)

    # named_modules order is the order the hooks fire in, which decides who owns a shared input
    linears = [(name, mod) for name, mod in model.named_modules() if isinstance(mod, nn.Linear) and wanted(name)]
    if not linears:
        raise ValueError("no Linear module matched only/skip")
    q_mods = dict(q_model.named_modules()) if q_model is not None else None

    probe = SharedInputProbe()
    handles = [mod.register_forward_pre_hook(probe.hook(name)) for name, mod in linears]
    try:
        with torch.no_grad():
            model(input_ids=samples[:1].to(dev), use_cache=False)  # one batch: identity does not depend on it
    finally:
        for h in handles:
            h.remove()
        probe.release()

    widths = {name: mod.in_features for name, mod in linears if name not in probe.alias_of}
    passes = plan_passes(widths, int(max_hessian_mem * GIB))
    paired = q_model is not None
    print(f"{len(linears)} Linear modules share {len(widths)} distinct inputs ({len(probe.alias_of)} aliases): "
          f"{human_size(sum(map(plan_entry_bytes, widths.values())))} planned in {len(passes)} pass(es)", file=log)

    nsamples = samples.shape[0]
    nbatches = (nsamples + batch - 1) // batch
    written = []
    for index, cp in enumerate(passes, 1):
        need = sum(device_entry_bytes(widths[o], paired) for o in cp.owners)
        free, _ = torch.cuda.mem_get_info(dev)
        if need > free:
            raise RuntimeError(f"capture pass {index}/{len(passes)} needs {human_size(need)} of f64 accumulators on "
                               f"the GPU, {human_size(free)} is free; lower max_hessian_mem")
        owners = set(cp.owners)
        acc = _PassAccumulators(ctx, dev, paired)
        handles = [mod.register_forward_pre_hook(acc.hook(name, "fp")) for name, mod in linears if name in owners]
        if paired:
            handles += [q_mods[name].register_forward_pre_hook(acc.hook(name, "q")) for name in cp.owners]
        try:
            with torch.no_grad():
                for b, s in enumerate(range(0, nsamples, batch), 1):
                    ids = samples[s:s + batch].to(dev)
                    acc.weights = (token_weight[ids].reshape(-1).float().contiguous()
                                   if token_weight is not None else None)
                    model(input_ids=ids, use_cache=False)
                    if paired:
                        q_model(input_ids=ids, use_cache=False)
                    print(f"pass {index}/{len(passes)}: batch {b}/{nbatches}", file=log)
        finally:
            for h in handles:
                h.remove()

        aliases = {dep: own for dep, own in probe.alias_of.items() if own in owners}
        tensors = acc.finalize()
        path = pass_file(out, index, len(passes))
        os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
        from safetensors.torch import save_file
        save_file(tensors, path, metadata=_header(acc.tokens, aliases))
        written.append(path)
        print(f"pass {index}/{len(passes)}: {len(acc.h)} Hessian(s), {len(aliases)} alias(es) -> {path}", file=log)
        del acc, tensors  # free this pass's accumulators before the next one
    return written

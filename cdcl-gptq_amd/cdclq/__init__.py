"""cdclq -- MI355X-native CDCL-GPTQ per-layer quantization engine (Python host binding).

Mirrors the reference crate's public engine API (tailot/CDCL-GPTQ `cdclq` 1.0.1):

    engine::Config / Method / LayerStats      src/engine.rs:83-199   -> Config, Method, LayerStats
    engine::quantize_layer(w, d_out, d_in, h, m, hkey, cfg, cache)
                                              src/engine.rs:690-699  -> quantize_layer(...)
    engine::PrepCache (Option<(String, Prepared)>)
                                              src/engine.rs:220-223  -> PrepCache (owns a GPU context)
    linalg::gram_accumulate(x, y, t, n, h)    src/linalg.rs:388      -> gram_accumulate(...)
    linalg::upper_chol_of_inverse(h, n)       src/linalg.rs:362      -> upper_chol_of_inverse(...)
    engine::proxy_loss                        src/engine.rs:808      -> proxy_loss(...)
    quant::QLayer (+ dequantize, bits_*)      src/quant.rs:161-250   -> QLayer

All computation runs in libcdclq_hip.so (hand-written gfx950 HIP kernels) through the C ABI in
include/cdclq.h. There is no CPU fallback: importing this module on a machine without the built
library, or calling it without a GPU, raises.
"""
from __future__ import annotations

import ctypes as C
import enum
import itertools
import os
from dataclasses import dataclass, field

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libcdclq_hip.so")

OK, INVALID_ARG, NOT_PD, NON_FINITE, DEVICE, OOM = range(6)
PHASE_GRAM, PHASE_FACTOR, PHASE_GPTQ, PHASE_REPAIR, PHASE_TARGET = range(5)
PHASE_NAMES = ["gram", "factor", "gptq", "repair", "target", "pack", "dequant"]


class CdclqError(RuntimeError):
    """Error raised by the engine. `code` is the cdclq_status value; the message is the
    reference's anyhow text where the reference reports the same condition."""

    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


class _Config(C.Structure):
    _fields_ = [
        ("bits", C.c_uint32), ("skeleton_bits", C.c_uint32), ("group", C.c_uint64), ("block", C.c_uint64),
        ("sub_block", C.c_uint64), ("cd_sweeps", C.c_uint64), ("passes", C.c_uint64), ("row_chunk", C.c_uint64),
        ("damp", C.c_double), ("skeleton_pct", C.c_double), ("refine_frac", C.c_double), ("tol", C.c_double),
        ("act_order", C.c_int32), ("mse_grid", C.c_int32), ("method", C.c_int32), ("refit_scales", C.c_int32),
    ]


class _Stats(C.Structure):
    _fields_ = [
        ("loss_gptq", C.c_double), ("loss_final", C.c_double), ("subblocks_total", C.c_uint64),
        ("subblocks_refined", C.c_uint64), ("code_updates", C.c_uint64), ("skeleton_groups", C.c_uint64),
        ("bits_codes", C.c_double), ("bits_total", C.c_double), ("secs_prepare", C.c_double),
        ("secs_quant", C.c_double),
    ]


class _BenchArgs(C.Structure):
    """bench::BenchArgs (src/bench.rs:19-32) + the rayon thread count."""

    _fields_ = [("rows", C.c_size_t), ("cols", C.c_size_t), ("tokens", C.c_size_t), ("test_tokens", C.c_size_t),
                ("seed", C.c_uint64), ("asym_noise", C.c_float), ("nthreads", C.c_uint32), ("cfg", _Config)]


class _BenchRow(C.Structure):
    """One report row (src/bench.rs:124-128)."""

    _fields_ = [("name", C.c_char * 96), ("loss", C.c_double), ("calib", C.c_double), ("test", C.c_double),
                ("secs", C.c_double), ("bpw", C.c_double)]


class _QuantOpts(C.Structure):
    """pipeline::QuantOpts (src/pipeline.rs:24-40) + thread count and verbosity."""

    _fields_ = [("weights", C.POINTER(C.c_char_p)), ("n_weights", C.c_size_t), ("hessians", C.POINTER(C.c_char_p)),
                ("n_hessians", C.c_size_t), ("out_dir", C.c_char_p), ("cfg", _Config),
                ("only", C.POINTER(C.c_char_p)), ("n_only", C.c_size_t), ("skip", C.POINTER(C.c_char_p)),
                ("n_skip", C.c_size_t), ("emit_packed", C.c_int32), ("emit_dequant", C.c_int32),
                ("nthreads", C.c_uint32), ("verbose", C.c_int32)]


_lib = None


def lib() -> C.CDLL:
    """The loaded libcdclq_hip.so (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it first (python -m cdclq.build or __graft_entry__.build())")
    L = C.CDLL(LIB_PATH)
    vp, sz, i32, u64 = C.c_void_p, C.c_size_t, C.c_int, C.c_uint64
    cfgp, stp = C.POINTER(_Config), C.POINTER(_Stats)
    sig = {
        "cdclq_abi_version": ([], i32),
        "cdclq_sizeof_config": ([], sz),
        "cdclq_sizeof_stats": ([], sz),
        "cdclq_default_config": ([cfgp], None),
        "cdclq_num_groups": ([cfgp, sz], sz),
        "cdclq_ctx_create": ([i32, C.POINTER(vp)], i32),
        "cdclq_ctx_destroy": ([vp], None),
        "cdclq_last_error": ([vp], C.c_char_p),
        "cdclq_ctx_clear_cache": ([vp], i32),
        "cdclq_quantize_layer": ([vp, vp, sz, sz, vp, vp, C.c_char_p, cfgp, sz, vp, vp, vp, vp, vp, stp], i32),
        "cdclq_quantize_layer_device": ([vp, vp, sz, sz, vp, vp, C.c_char_p, cfgp, sz, vp, vp, vp, vp, vp, stp], i32),
        "cdclq_prepare_layer_device": ([vp, vp, sz, sz, vp, C.c_char_p, cfgp], i32),
        "cdclq_gram_accumulate": ([vp, vp, vp, sz, sz, vp], i32),
        "cdclq_gram_accumulate_device": ([vp, vp, vp, sz, sz, vp], i32),
        "cdclq_gram_accumulate_device_noalloc": ([vp, vp, vp, sz, sz, vp], i32),
        "cdclq_ctx_last_midpoint_counts": ([vp, vp], i32),
        "cdclq_sgemm_device": ([vp, sz, sz, sz, C.c_float, vp, C.c_ssize_t, C.c_ssize_t, vp, C.c_ssize_t,
                                C.c_ssize_t, C.c_float, vp, C.c_ssize_t, C.c_ssize_t], i32),
        "cdclq_dgemm_device": ([vp, sz, sz, sz, C.c_double, vp, C.c_ssize_t, C.c_ssize_t, vp, C.c_ssize_t,
                                C.c_ssize_t, C.c_double, vp, C.c_ssize_t, C.c_ssize_t], i32),
        "cdclq_gram_accumulate_batch_device": ([vp, i32, C.POINTER(vp), C.POINTER(vp), C.POINTER(sz), C.POINTER(sz),
                                                C.POINTER(vp)], i32),
        "cdclq_upper_chol_of_inverse": ([vp, vp, sz, vp], i32),
        "cdclq_upper_chol_of_inverse_device": ([vp, vp, sz, vp], i32),
        "cdclq_proxy_loss": ([vp, vp, vp, sz, sz, vp, C.POINTER(C.c_double)], i32),
        "cdclq_row_bytes": ([sz, sz, vp, sz, C.POINTER(sz)], i32),
        "cdclq_pack_layer": ([vp, sz, sz, sz, vp, sz, vp, vp, vp, vp, vp, sz, vp, vp, vp], i32),
        "cdclq_pack_layer_device": ([vp, sz, sz, sz, vp, sz, vp, vp, vp, vp, vp, sz, vp, vp, vp], i32),
        "cdclq_dequantize_packed": ([vp, sz, sz, sz, vp, sz, vp, sz, vp, vp, vp, i32, vp], i32),
        "cdclq_dequantize_packed_device": ([vp, sz, sz, sz, vp, sz, vp, sz, vp, vp, vp, i32, vp], i32),
        "cdclq_dequantize_layer": ([vp, sz, sz, sz, sz, vp, vp, vp, vp, i32, vp], i32),
        "cdclq_dequantize_layer_device": ([vp, sz, sz, sz, sz, vp, vp, vp, vp, i32, vp], i32),
        "cdclq_rtn_layer": ([vp, vp, sz, sz, cfgp, vp], i32),
        "cdclq_rtn_layer_device": ([vp, vp, sz, sz, cfgp, vp], i32),
        "cdclq_proxy_loss_device": ([vp, vp, vp, sz, sz, vp, C.POINTER(C.c_double)], i32),
        "cdclq_rel_err": ([vp, vp, vp, vp, vp, sz, sz, sz, C.POINTER(C.c_double)], i32),
        "cdclq_rel_err_device": ([vp, vp, vp, vp, vp, sz, sz, sz, C.POINTER(C.c_double)], i32),
        "cdclq_bench_run": ([vp, C.POINTER(_BenchArgs), C.POINTER(_BenchRow), sz, C.POINTER(sz), C.c_char_p, sz,
                             C.POINTER(sz)], i32),
        "cdclq_quantize_model": ([vp, C.POINTER(_QuantOpts), C.c_char_p, sz, C.POINTER(sz)], i32),
        "cdclq_dequantize_model": ([vp, C.c_char_p, C.c_char_p, i32, C.POINTER(sz)], i32),
        "cdclq_hessian_accumulate_device": ([vp, vp, vp, vp, sz, sz, vp], i32),
        "cdclq_hessian_finalize_device": ([vp, vp, sz, u64, vp], i32),
        "cdclq_device_alloc": ([vp, sz, C.POINTER(vp)], i32),
        "cdclq_device_free": ([vp, vp], i32),
        "cdclq_memcpy_h2d": ([vp, vp, vp, sz], i32),
        "cdclq_memcpy_d2h": ([vp, vp, vp, sz], i32),
        "cdclq_memset_device": ([vp, vp, i32, sz], i32),
        "cdclq_synth_normal_device": ([vp, u64, u64, sz, C.c_float, vp], i32),
        "cdclq_synth_outlier_scales": ([u64, sz, C.c_double, C.c_float, vp], i32),
        "cdclq_synth_tokens_device": ([vp, u64, u64, sz, sz, vp, vp], i32),
        "cdclq_synth_tokens_heavy_device": ([vp, u64, u64, sz, sz, vp, vp, vp], i32),
        "cdclq_synth_perturb_device": ([vp, u64, u64, sz, C.c_float, vp, vp], i32),
        "cdclq_synth_lognormal_scales": ([u64, sz, C.c_float, vp], i32),
        "cdclq_f64_to_f32_device": ([vp, vp, sz, vp], i32),
        "cdclq_ctx_set_timing": ([vp, i32], i32),
        "cdclq_ctx_reset_timing": ([vp], i32),
        "cdclq_ctx_get_timing": ([vp, i32, C.POINTER(C.c_uint64), C.POINTER(C.c_double)], i32),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    _lib = L
    return L


EXPORTED_SYMBOLS = None  # filled lazily by exported_symbols()


def exported_symbols() -> list[str]:
    """Names of the C-ABI entry points this binding expects the library to export."""
    return [
        "cdclq_abi_version", "cdclq_sizeof_config", "cdclq_sizeof_stats", "cdclq_default_config",
        "cdclq_num_groups", "cdclq_ctx_create", "cdclq_ctx_destroy", "cdclq_last_error", "cdclq_ctx_clear_cache",
        "cdclq_quantize_layer", "cdclq_quantize_layer_device", "cdclq_prepare_layer_device", "cdclq_gram_accumulate",
        "cdclq_gram_accumulate_device", "cdclq_gram_accumulate_device_noalloc", "cdclq_gram_accumulate_batch_device",
        "cdclq_sgemm_device", "cdclq_dgemm_device", "cdclq_ctx_last_midpoint_counts", "cdclq_upper_chol_of_inverse", "cdclq_upper_chol_of_inverse_device",
        "cdclq_proxy_loss", "cdclq_device_alloc", "cdclq_device_free", "cdclq_memcpy_h2d", "cdclq_memcpy_d2h",
        "cdclq_memset_device", "cdclq_synth_normal_device", "cdclq_synth_outlier_scales", "cdclq_synth_tokens_device",
        "cdclq_synth_tokens_heavy_device", "cdclq_synth_perturb_device", "cdclq_synth_lognormal_scales",
        "cdclq_f64_to_f32_device",
        "cdclq_ctx_set_timing", "cdclq_ctx_reset_timing", "cdclq_ctx_get_timing",
        "cdclq_row_bytes", "cdclq_pack_layer", "cdclq_pack_layer_device", "cdclq_dequantize_packed",
        "cdclq_dequantize_packed_device", "cdclq_dequantize_layer", "cdclq_dequantize_layer_device",
        "cdclq_rtn_layer", "cdclq_rtn_layer_device", "cdclq_proxy_loss_device", "cdclq_rel_err",
        "cdclq_rel_err_device", "cdclq_bench_run", "cdclq_quantize_model", "cdclq_dequantize_model",
        "cdclq_hessian_accumulate_device", "cdclq_hessian_finalize_device",
    ]


MIDPOINT_FIELDS = ("code_decisions", "code_near", "zero_decisions", "zero_near", "cd_decisions", "cd_near")


class Method(enum.IntEnum):
    """engine::Method (src/engine.rs:83-88)."""

    Gptq = 0
    Cdcl = 1


@dataclass
class Config:
    """engine::Config with the reference defaults (src/engine.rs:94-167)."""

    bits: int = 3
    group: int = 128
    block: int = 128
    damp: float = 0.01
    act_order: bool = True
    skeleton_pct: float = 0.0
    skeleton_bits: int = 8
    mse_grid: bool = False
    method: Method = Method.Cdcl
    refine_frac: float = 1.0
    sub_block: int = 64
    cd_sweeps: int = 1
    passes: int = 10
    tol: float = 1e-3
    refit_scales: bool = True
    row_chunk: int = 0

    def _c(self) -> _Config:
        c = _Config()
        for name, _ in _Config._fields_:
            v = getattr(self, name)
            setattr(c, name, int(v) if isinstance(v, (bool, enum.Enum)) else v)
        return c


def effective_group(cfg: Config, n: int) -> int:
    """engine::effective_group (src/engine.rs:227-233)."""
    return n if (cfg.group == 0 or cfg.group >= n) else cfg.group


@dataclass
class LayerStats:
    """engine::LayerStats (src/engine.rs:174-199)."""

    loss_gptq: float = 0.0
    loss_final: float = 0.0
    subblocks_total: int = 0
    subblocks_refined: int = 0
    code_updates: int = 0
    skeleton_groups: int = 0
    bits_codes: float = 0.0
    bits_total: float = 0.0
    secs_prepare: float = 0.0
    secs_quant: float = 0.0


@dataclass
class QLayer:
    """quant::QLayer (src/quant.rs:161-175): codes in permuted column order."""

    d_out: int
    d_in: int
    group: int
    perm: np.ndarray
    gbits: np.ndarray
    codes: np.ndarray
    scales: np.ndarray
    zeros: np.ndarray

    def ngroups(self) -> int:
        return int(self.gbits.size)

    def dequantize(self) -> np.ndarray:
        """QLayer::dequantize (src/quant.rs:189-202): original column order."""
        g = self.group
        gi = np.arange(self.d_in) // g
        vals = self.scales[:, gi] * (self.codes.astype(np.float32) - self.zeros[:, gi])
        out = np.zeros((self.d_out, self.d_in), np.float32)
        out[:, self.perm.astype(np.int64)] = vals
        return out

    def bits_codes(self) -> float:
        return float(self.gbits[np.arange(self.d_in) // self.group].astype(np.int64).sum()) / self.d_in

    def bits_total(self) -> float:
        return self.bits_codes() + 24.0 / self.group


def _check(ctx_ptr, rc: int):
    if rc != OK:
        msg = lib().cdclq_last_error(ctx_ptr)
        raise CdclqError(rc, msg.decode() if msg else f"cdclq error {rc}")


class Context:
    """A GPU context: HIP stream, device workspace and the one-entry factor cache."""

    def __init__(self, device: int = 0):
        L = lib()
        p = C.c_void_p()
        rc = L.cdclq_ctx_create(device, C.byref(p))
        if rc != OK:
            raise CdclqError(rc, f"cdclq_ctx_create(device={device}) failed (no usable GPU?)")
        self.ptr = p
        self.device = device
        self.cache_owner = None  # token of the PrepCache whose entry the context's factor cache holds

    def close(self):
        if getattr(self, "ptr", None) and _lib is not None:
            _lib.cdclq_ctx_destroy(self.ptr)
            self.ptr = None

    def __del__(self):
        self.close()

    def check(self, rc: int):
        _check(self.ptr, rc)

    def clear_cache(self):
        self.check(lib().cdclq_ctx_clear_cache(self.ptr))
        self.cache_owner = None

    def last_midpoint_counts(self) -> dict:
        """Near-midpoint accounting of the last quantize_layer call on this context
        (cdclq_midpoint_counts in include/cdclq.h)."""
        mc = (C.c_uint64 * 6)()
        self.check(lib().cdclq_ctx_last_midpoint_counts(self.ptr, mc))
        return dict(zip(MIDPOINT_FIELDS, (int(v) for v in mc)))

    # ---- timing
    def set_timing(self, on: bool):
        self.check(lib().cdclq_ctx_set_timing(self.ptr, int(on)))

    def reset_timing(self):
        self.check(lib().cdclq_ctx_reset_timing(self.ptr))

    def timing(self) -> dict:
        out = {}
        for i, name in enumerate(PHASE_NAMES):
            n, ms = C.c_uint64(), C.c_double()
            self.check(lib().cdclq_ctx_get_timing(self.ptr, i, C.byref(n), C.byref(ms)))
            out[name] = {"launches": n.value, "ms": ms.value}
        return out


class PrepCache:
    """engine::PrepCache handle: callers create it empty and pass it to every quantize_layer call
    (src/engine.rs:220-223). The factorisation itself lives in the context's one-entry cache; a
    context shared by several PrepCache objects serves each of them as its own cache: the entry
    belongs to the cache that filled it, and a call through another cache drops it first. So a new
    PrepCache is always empty, like `None` in the reference, even when it reuses a context."""

    _tokens = itertools.count(1)

    def __init__(self, device: int = 0, ctx: Context | None = None):
        self.ctx = ctx or Context(device)
        self.token = next(PrepCache._tokens)

    def claim(self) -> Context:
        """The context, with its cache entry dropped unless this cache filled it."""
        if self.ctx.cache_owner != self.token:
            self.ctx.clear_cache()
            self.ctx.cache_owner = self.token
        return self.ctx


class DeviceArray:
    """A device (HBM) buffer owned through the C ABI, with numpy-typed upload/download."""

    def __init__(self, ctx: Context, shape, dtype):
        self.ctx = ctx
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = C.c_void_p()
        ctx.check(lib().cdclq_device_alloc(ctx.ptr, self.nbytes, C.byref(p)))
        self.ptr = p

    @classmethod
    def from_host(cls, ctx: Context, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(ctx, a.shape, a.dtype)
        d.upload(a)
        return d

    @property
    def addr(self) -> int:
        return int(self.ptr.value or 0)

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a, self.dtype)
        assert a.nbytes == self.nbytes
        self.ctx.check(lib().cdclq_memcpy_h2d(self.ctx.ptr, self.ptr, a.ctypes.data, self.nbytes))

    def download(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        self.ctx.check(lib().cdclq_memcpy_d2h(self.ctx.ptr, out.ctypes.data, self.ptr, self.nbytes))
        return out

    def zero(self):
        self.ctx.check(lib().cdclq_memset_device(self.ctx.ptr, self.ptr, 0, self.nbytes))

    def free(self):
        if getattr(self, "ptr", None) is not None and self.ptr.value and _lib is not None and self.ctx.ptr:
            _lib.cdclq_device_free(self.ctx.ptr, self.ptr)
        self.ptr = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32)


def quantize_layer(w, d_out: int, d_in: int, h, m, hkey: str, cfg: Config, cache: PrepCache,
                   nthreads: int = 24) -> tuple[QLayer, LayerStats]:
    """engine::quantize_layer (src/engine.rs:690-799) on the GPU. `w` (d_out x d_in) and `h`
    (d_in x d_in) are host arrays (f32); `m` is the optional cross-covariance or None.
    `nthreads` stands in for rayon::current_num_threads() when cfg.row_chunk == 0."""
    w = _f32(w).reshape(d_out, d_in)
    h = _f32(h).reshape(d_in, d_in)
    if m is not None:
        m = _f32(m).reshape(d_in, d_in)
    ctx = cache.claim()
    n = d_in
    g = effective_group(cfg, n)
    ng = (n + g - 1) // g
    codes = np.zeros((d_out, n), np.uint8)
    scales = np.zeros((d_out, ng), np.float32)
    zeros = np.zeros((d_out, ng), np.float32)
    perm = np.zeros(n, np.uint32)
    gbits = np.zeros(ng, np.uint8)
    st = _Stats()
    c = cfg._c()
    rc = lib().cdclq_quantize_layer(ctx.ptr, w.ctypes.data, d_out, n, h.ctypes.data,
                                    m.ctypes.data if m is not None else None, hkey.encode(), C.byref(c), nthreads,
                                    codes.ctypes.data, scales.ctypes.data, zeros.ctypes.data, perm.ctypes.data,
                                    gbits.ctypes.data, C.byref(st))
    ctx.check(rc)
    stats = LayerStats(**{f: getattr(st, f) for f, _ in _Stats._fields_})
    return QLayer(d_out, n, g, perm, gbits, codes, scales, zeros), stats


def quantize_layer_device(ctx: Context, w: DeviceArray, d_out: int, d_in: int, h: DeviceArray,
                          m: DeviceArray | None, hkey: str, cfg: Config, codes: DeviceArray, scales: DeviceArray,
                          zeros: DeviceArray, nthreads: int = 24):
    """Device-resident variant: inputs and codes/scales/zeros stay in HBM. Returns (perm, gbits,
    LayerStats) on the host."""
    n = d_in
    g = effective_group(cfg, n)
    ng = (n + g - 1) // g
    perm = np.zeros(n, np.uint32)
    gbits = np.zeros(ng, np.uint8)
    st = _Stats()
    c = cfg._c()
    ctx.check(lib().cdclq_quantize_layer_device(ctx.ptr, w.ptr, d_out, n, h.ptr, m.ptr if m is not None else None,
                                                hkey.encode(), C.byref(c), nthreads, codes.ptr, scales.ptr,
                                                zeros.ptr, perm.ctypes.data, gbits.ctypes.data, C.byref(st)))
    return perm, gbits, LayerStats(**{f: getattr(st, f) for f, _ in _Stats._fields_})


def prepare_layer_device(ctx: Context, w: DeviceArray, d_out: int, d_in: int, h: DeviceArray, hkey: str,
                         cfg: Config):
    """The factor cache fill of quantize_layer on its own (src/engine.rs:708-723): a following
    quantize_layer_device on ctx with the same hkey, h and cfg reuses it."""
    ctx.check(lib().cdclq_prepare_layer_device(ctx.ptr, w.ptr, d_out, d_in, h.ptr, hkey.encode(), C.byref(cfg._c())))


def gram_accumulate(x, y, t: int, n: int, h: np.ndarray, ctx: Context) -> np.ndarray:
    """linalg::gram_accumulate (src/linalg.rs:388-418): h (f64, n x n) += x^T y, in place.
    Pass the same array object for x and y for the symmetric Hessian."""
    sym = y is x
    x = _f32(x).reshape(t, n)
    y = x if sym else _f32(y).reshape(t, n)
    assert h.dtype == np.float64 and h.shape == (n, n) and h.flags.c_contiguous
    ctx.check(lib().cdclq_gram_accumulate(ctx.ptr, x.ctypes.data, y.ctypes.data, t, n, h.ctypes.data))
    return h


def gram_accumulate_batch_device(ctx: Context, xs, ys, ts, ns, hs):
    """Several device-resident accumulations hs[i] += xs[i]^T ys[i] in one launch."""
    k = len(xs)
    arr = lambda v: (C.c_void_p * k)(*[a.ptr.value for a in v])
    ctx.check(lib().cdclq_gram_accumulate_batch_device(ctx.ptr, k, arr(xs), arr(ys), (C.c_size_t * k)(*ts),
                                                        (C.c_size_t * k)(*ns), arr(hs)))


def upper_chol_of_inverse(h64, n: int, ctx: Context) -> np.ndarray:
    """linalg::upper_chol_of_inverse (src/linalg.rs:362-375)."""
    h64 = np.ascontiguousarray(h64, np.float64).reshape(n, n)
    u = np.zeros((n, n), np.float32)
    ctx.check(lib().cdclq_upper_chol_of_inverse(ctx.ptr, h64.ctypes.data, n, u.ctypes.data))
    return u


def proxy_loss(w_t, w_hat, rows: int, n: int, h, ctx: Context) -> float:
    """engine::proxy_loss (src/engine.rs:808-815)."""
    w_t, w_hat, h = _f32(w_t), _f32(w_hat), _f32(h)
    out = C.c_double()
    ctx.check(lib().cdclq_proxy_loss(ctx.ptr, w_t.ctypes.data, w_hat.ctypes.data, rows, n, h.ctypes.data,
                                     C.byref(out)))
    return out.value


def synth_outlier_scales(seed: int, n: int, frac: float, factor: float) -> np.ndarray:
    """Channel-scale vector of the synthetic calibration inputs (see include/cdclq.h)."""
    out = np.empty(n, np.float32)
    rc = lib().cdclq_synth_outlier_scales(seed, n, frac, factor, out.ctypes.data)
    if rc != OK:
        raise CdclqError(rc, "cdclq_synth_outlier_scales failed")
    return out


def synth_heavy_channels(seed: int, n: int, frac: float) -> np.ndarray:
    """Mask of round(frac * n) channels (the seeded pick of synth_outlier_scales) that draw
    Student-t(3) values in synth_tokens_device."""
    return (synth_outlier_scales(seed, n, frac, 2.0) != 1.0).astype(np.uint8)


def synth_lognormal_scales(seed: int, n: int, sigma: float) -> np.ndarray:
    """exp(sigma * normal(seed, j)) per channel j (log-normal channel scales)."""
    out = np.empty(n, np.float32)
    rc = lib().cdclq_synth_lognormal_scales(seed, n, sigma, out.ctypes.data)
    if rc != OK:
        raise CdclqError(rc, "cdclq_synth_lognormal_scales failed")
    return out


def synth_tokens_device(ctx: "Context", seed: int, t: int, n: int, x: "DeviceArray", ch_scale=None, heavy=None,
                        row0: int = 0):
    """x (t x n, device) = counter-based tokens; ch_scale: n f32 channel scales, heavy: n-channel
    mask of Student-t(3) channels (both host arrays or None)."""
    cs = None if ch_scale is None else np.ascontiguousarray(ch_scale, np.float32)
    hv = None if heavy is None else np.ascontiguousarray(heavy, np.uint8)
    ctx.check(lib().cdclq_synth_tokens_heavy_device(ctx.ptr, seed, row0, t, n, None if cs is None else cs.ctypes.data,
                                                    None if hv is None else hv.ctypes.data, x.ptr))


def synth_perturb_device(ctx: "Context", seed: int, x: "DeviceArray", out: "DeviceArray", sigma: float,
                         offset: int = 0):
    """out = x + sigma * N(0, 1) (counter stream `seed`), elementwise on the device."""
    count = int(np.prod(x.shape))
    ctx.check(lib().cdclq_synth_perturb_device(ctx.ptr, seed, offset, count, sigma, x.ptr, out.ptr))


# ---------------------------------------------------------------- packed container cdclq-v1
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
_DTYPE_CODE = {"F32": DTYPE_F32, "F16": DTYPE_F16, "BF16": DTYPE_BF16}
_DTYPE_NP = {DTYPE_F32: np.float32, DTYPE_F16: np.uint16, DTYPE_BF16: np.uint16}


def _dtype_code(dtype) -> int:
    return _DTYPE_CODE[dtype.upper()] if isinstance(dtype, str) else int(dtype)


def row_bytes(n: int, g: int, gbits) -> int:
    """quant::row_bytes (src/quant.rs:102-104)."""
    gbits = np.ascontiguousarray(gbits, np.uint8)
    out = C.c_size_t()
    rc = lib().cdclq_row_bytes(n, g, gbits.ctypes.data, gbits.size, C.byref(out))
    if rc != OK:
        raise CdclqError(rc, f"invalid packed layout (n={n}, group={g}, gbits={gbits.tolist()[:8]}...)")
    return out.value


def pack_layer(ctx: Context, ql: QLayer):
    """QLayer::pack + io::packed_tensors (src/quant.rs:207-214, src/io.rs:244-264) on the GPU:
    (qweight u8 [d_out, row_bytes], scales f16 bits u16 [d_out, ng], qzeros u8 [d_out, ng],
    perm i32 [d_in])."""
    gbits = np.ascontiguousarray(ql.gbits, np.uint8)
    ng = gbits.size
    rb = row_bytes(ql.d_in, ql.group, gbits)
    codes = np.ascontiguousarray(ql.codes, np.uint8)
    scales, zeros = _f32(ql.scales), _f32(ql.zeros)
    perm = np.ascontiguousarray(ql.perm, np.uint32)
    qw = np.zeros((ql.d_out, rb), np.uint8)
    s16 = np.zeros((ql.d_out, ng), np.uint16)
    qz = np.zeros((ql.d_out, ng), np.uint8)
    p32 = np.zeros(ql.d_in, np.int32)
    ctx.check(lib().cdclq_pack_layer(ctx.ptr, ql.d_out, ql.d_in, ql.group, gbits.ctypes.data, ng, codes.ctypes.data,
                                     scales.ctypes.data, zeros.ctypes.data, perm.ctypes.data, qw.ctypes.data, qw.size,
                                     s16.ctypes.data, qz.ctypes.data, p32.ctypes.data))
    return qw, s16, qz, p32


def packed_tensors(layer: str, ql: QLayer, ctx: Context) -> dict:
    """io::packed_tensors (src/io.rs:244-264): the six tensors of one packed layer, name ->
    (safetensors dtype, numpy array). F16 scales are carried as their uint16 bit patterns."""
    qw, s16, qz, p32 = pack_layer(ctx, ql)
    return {
        f"{layer}.qweight": ("U8", qw),
        f"{layer}.scales": ("F16", s16),
        f"{layer}.qzeros": ("U8", qz),
        f"{layer}.perm": ("I32", p32),
        f"{layer}.gbits": ("U8", np.ascontiguousarray(ql.gbits, np.uint8).copy()),
        f"{layer}.gsize": ("I32", np.array([ql.group], np.int32)),
    }


def dequantize_packed(ctx: Context, qweight, scales_f16, qzeros, perm_i32, gbits, group: int, dtype="F32"):
    """io::read_packed_layer + QLayer::dequantize + io::f32_to_bytes (src/io.rs:270-293,
    src/quant.rs:189-236, src/io.rs:50-57) on the GPU. Returns d_out x d_in in the original column
    order: float32 for F32, uint16 bit patterns for F16 / BF16."""
    dt = _dtype_code(dtype)
    qweight = np.ascontiguousarray(qweight, np.uint8)
    s16 = np.ascontiguousarray(scales_f16, np.uint16)
    qz = np.ascontiguousarray(qzeros, np.uint8)
    p32 = np.ascontiguousarray(perm_i32, np.int32)
    gbits = np.ascontiguousarray(gbits, np.uint8)
    d_out, d_in = qweight.shape[0], p32.size
    out = np.zeros((d_out, d_in), _DTYPE_NP.get(dt, np.float32))
    ctx.check(lib().cdclq_dequantize_packed(ctx.ptr, d_out, d_in, group, gbits.ctypes.data, gbits.size,
                                            qweight.ctypes.data, qweight.size, s16.ctypes.data, qz.ctypes.data,
                                            p32.ctypes.data, dt, out.ctypes.data))
    return out


def read_packed_dequantized(tensors: dict, layer: str, ctx: Context, dtype="F32"):
    """The `cdclq dequant` expansion of one layer (src/pipeline.rs:239-262) from a dict in the
    packed_tensors() form; a missing companion tensor raises with its name (src/io.rs:271-274)."""
    def get(suffix):
        key = f"{layer}.{suffix}"
        if key not in tensors:
            raise KeyError(f"{key}: missing")
        v = tensors[key]
        return v[1] if isinstance(v, tuple) else v
    qw, s16, qz, p32, gb, gs = (get(x) for x in ("qweight", "scales", "qzeros", "perm", "gbits", "gsize"))
    return dequantize_packed(ctx, qw, s16, qz, p32, gb, int(np.asarray(gs).ravel()[0]), dtype)


def dequantize_layer(ctx: Context, ql: QLayer, dtype="F32"):
    """QLayer::dequantize + io::f32_to_bytes (src/quant.rs:189-202, src/io.rs:50-57) on the GPU."""
    dt = _dtype_code(dtype)
    codes = np.ascontiguousarray(ql.codes, np.uint8)
    scales, zeros = _f32(ql.scales), _f32(ql.zeros)
    perm = np.ascontiguousarray(ql.perm, np.uint32)
    out = np.zeros((ql.d_out, ql.d_in), _DTYPE_NP.get(dt, np.float32))
    ctx.check(lib().cdclq_dequantize_layer(ctx.ptr, ql.d_out, ql.d_in, ql.group, int(np.asarray(ql.gbits).size),
                                           codes.ctypes.data, scales.ctypes.data, zeros.ctypes.data, perm.ctypes.data,
                                           dt, out.ctypes.data))
    return out


# ---------------------------------------------------------------- evaluation / synthetic benchmark
def rtn_layer(ctx: Context, w, cfg: Config) -> np.ndarray:
    """engine::rtn_layer (src/engine.rs:822-838) on the GPU."""
    w = _f32(w)
    out = np.zeros_like(w)
    c = cfg._c()
    ctx.check(lib().cdclq_rtn_layer(ctx.ptr, w.ctypes.data, w.shape[0], w.shape[1], C.byref(c), out.ctypes.data))
    return out


def rel_err(ctx: Context, w, w_hat, x, x_t=None) -> float:
    """bench::rel_err (src/bench.rs:106-121): ||W x - W_hat x~||^2 / ||W x||^2 (x: t x n tokens)."""
    w, w_hat, x = _f32(w), _f32(w_hat), _f32(x)
    xt = x if x_t is None else _f32(x_t)
    out = C.c_double()
    ctx.check(lib().cdclq_rel_err(ctx.ptr, w.ctypes.data, w_hat.ctypes.data, x.ctypes.data, xt.ctypes.data,
                                  w.shape[0], w.shape[1], x.shape[0], C.byref(out)))
    return out.value


@dataclass
class BenchRow:
    name: str
    loss: float
    calib: float
    test: float
    secs: float
    bpw: float


def bench_run(ctx: Context, cfg: Config, rows: int = 1024, cols: int = 2048, tokens: int = 16384,
              test_tokens: int = 4096, seed: int = 1, asym_noise: float = 0.0, nthreads: int = 1):
    """bench::run (src/bench.rs:164-340) on the GPU: (markdown report, [BenchRow]). Defaults are the
    `cdclq bench` CLI defaults (src/main.rs:171-190)."""
    a = _BenchArgs(rows=rows, cols=cols, tokens=tokens, test_tokens=test_tokens, seed=seed, asym_noise=asym_noise,
                   nthreads=nthreads, cfg=cfg._c())
    cap_rows = 32
    out = (_BenchRow * cap_rows)()
    nrows, rlen = C.c_size_t(), C.c_size_t()
    buf = C.create_string_buffer(1 << 16)
    ctx.check(lib().cdclq_bench_run(ctx.ptr, C.byref(a), out, cap_rows, C.byref(nrows), buf, len(buf), C.byref(rlen)))
    res = [BenchRow(out[i].name.decode(), out[i].loss, out[i].calib, out[i].test, out[i].secs, out[i].bpw)
           for i in range(min(nrows.value, cap_rows))]
    return buf.value.decode(), res


# ---------------------------------------------------------------- model pipeline
def _cstrs(items):
    items = [str(x).encode() for x in items]
    return (C.c_char_p * max(len(items), 1))(*items), len(items)


def quantize_model(ctx: Context, weights, hessians, out_dir, cfg: Config, only=(), skip=(), emit_packed: bool = True,
                   emit_dequant: bool = True, nthreads: int = 24, verbose: bool = False) -> dict:
    """pipeline::quantize_model (src/pipeline.rs:79-227) on the GPU; returns the parsed report.json."""
    import json
    w, nw = _cstrs(weights)
    h, nh = _cstrs(hessians)
    on, non = _cstrs(only)
    sk, nsk = _cstrs(skip)
    o = _QuantOpts(weights=w, n_weights=nw, hessians=h, n_hessians=nh, out_dir=str(out_dir).encode(), cfg=cfg._c(),
                   only=on, n_only=non, skip=sk, n_skip=nsk, emit_packed=int(emit_packed),
                   emit_dequant=int(emit_dequant), nthreads=nthreads, verbose=int(verbose))
    need = C.c_size_t()
    buf = C.create_string_buffer(1 << 20)
    ctx.check(lib().cdclq_quantize_model(ctx.ptr, C.byref(o), buf, len(buf), C.byref(need)))
    if need.value >= len(buf):
        with open(os.path.join(str(out_dir), "report.json")) as f:
            return json.load(f)
    return json.loads(buf.value.decode())


def dequantize_model(ctx: Context, input_path, output_path, dtype=None) -> int:
    """pipeline::dequantize_packed (src/pipeline.rs:239-275): expands a packed shard; returns the
    number of layers. dtype None = the header's orig_dtype (else F16)."""
    n = C.c_size_t()
    dt = -1 if dtype is None else _dtype_code(dtype)
    ctx.check(lib().cdclq_dequantize_model(ctx.ptr, str(input_path).encode(), str(output_path).encode(), dt,
                                           C.byref(n)))
    return n.value


def default_config() -> Config:
    return Config()

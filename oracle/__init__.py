"""ctypes binding of the CPU oracle (oracle/cdclq_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker. The product library never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libcdclq_oracle.so")


class OrcConfig(C.Structure):
    """Field layout of orc_config / cdclq_config (src/engine.rs:94-144)."""

    _fields_ = [
        ("bits", C.c_uint32),
        ("skeleton_bits", C.c_uint32),
        ("group", C.c_uint64),
        ("block", C.c_uint64),
        ("sub_block", C.c_uint64),
        ("cd_sweeps", C.c_uint64),
        ("passes", C.c_uint64),
        ("row_chunk", C.c_uint64),
        ("damp", C.c_double),
        ("skeleton_pct", C.c_double),
        ("refine_frac", C.c_double),
        ("tol", C.c_double),
        ("act_order", C.c_int32),
        ("mse_grid", C.c_int32),
        ("method", C.c_int32),
        ("refit_scales", C.c_int32),
    ]


class OrcStats(C.Structure):
    """engine::LayerStats (src/engine.rs:174-199)."""

    _fields_ = [
        ("loss_gptq", C.c_double),
        ("loss_final", C.c_double),
        ("subblocks_total", C.c_uint64),
        ("subblocks_refined", C.c_uint64),
        ("code_updates", C.c_uint64),
        ("skeleton_groups", C.c_uint64),
        ("bits_codes", C.c_double),
        ("bits_total", C.c_double),
        ("secs_prepare", C.c_double),
        ("secs_quant", C.c_double),
    ]

    def as_dict(self):
        return {f: getattr(self, f) for f, _ in self._fields_}


def build(force: bool = False) -> str:
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
        f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
        u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
        u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
        sz = C.c_size_t
        pd = C.c_ssize_t
        L.orc_sizeof_config.restype = sz
        L.orc_sizeof_stats.restype = sz
        L.orc_default_config.argtypes = [C.POINTER(OrcConfig)]
        L.orc_round_f16.argtypes = [C.c_float]
        L.orc_round_f16.restype = C.c_float
        L.orc_round_f16_array.argtypes = [f32p, f32p, sz]
        L.orc_find_params.argtypes = [f32p, sz, C.c_uint32, C.c_int, C.POINTER(C.c_float), C.POINTER(C.c_float)]
        L.orc_quant_code.argtypes = [C.c_float, C.c_float, C.c_float, C.c_float, C.POINTER(C.c_uint8)]
        L.orc_quant_code.restype = C.c_float
        L.orc_sgemm.argtypes = [sz, sz, sz, C.c_float, C.c_void_p, pd, pd, C.c_void_p, pd, pd, C.c_float, C.c_void_p, pd, pd]
        L.orc_dgemm.argtypes = [sz, sz, sz, C.c_double, C.c_void_p, pd, pd, C.c_void_p, pd, pd, C.c_double, C.c_void_p, pd, pd]
        L.orc_cholesky_lower.argtypes = [f64p, sz, C.c_char_p, sz]
        L.orc_cholesky_lower.restype = C.c_int
        L.orc_tri_inverse_lower.argtypes = [f64p, sz, f64p]
        L.orc_upper_chol_of_inverse.argtypes = [f64p, sz, f32p, C.c_char_p, sz]
        L.orc_upper_chol_of_inverse.restype = C.c_int
        L.orc_gram_accumulate.argtypes = [f32p, f32p, sz, sz, f64p]
        L.orc_cache_new.restype = C.c_void_p
        L.orc_cache_free.argtypes = [C.c_void_p]
        L.orc_quantize_layer.argtypes = [f32p, sz, sz, f32p, C.c_void_p, C.c_char_p, C.POINTER(OrcConfig), sz, C.c_void_p,
                                         u8p, f32p, f32p, u32p, u8p, C.POINTER(OrcStats), C.c_char_p, sz]
        L.orc_quantize_layer.restype = C.c_int
        L.orc_num_groups.argtypes = [C.POINTER(OrcConfig), sz]
        L.orc_num_groups.restype = sz
        L.orc_proxy_loss.argtypes = [f32p, f32p, sz, sz, f32p]
        L.orc_proxy_loss.restype = C.c_double
        L.orc_rtn_layer.argtypes = [f32p, sz, sz, C.POINTER(OrcConfig), f32p]
        L.orc_dequantize.argtypes = [sz, sz, sz, u32p, sz, u8p, f32p, f32p, f32p]
        u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
        i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
        L.orc_f32_to_f16_bits.argtypes = [C.c_float]
        L.orc_f32_to_f16_bits.restype = C.c_uint16
        L.orc_f16_bits_to_f32.argtypes = [C.c_uint16]
        L.orc_f16_bits_to_f32.restype = C.c_float
        L.orc_f32_to_bf16_bits.argtypes = [C.c_float]
        L.orc_f32_to_bf16_bits.restype = C.c_uint16
        L.orc_narrow.argtypes = [f32p, sz, C.c_int, C.c_void_p]
        L.orc_row_bytes.argtypes = [sz, sz, u8p]
        L.orc_row_bytes.restype = sz
        L.orc_pack_row.argtypes = [u8p, sz, sz, u8p, u8p]
        L.orc_unpack_row.argtypes = [u8p, sz, sz, u8p, u8p]
        L.orc_pack_layer.argtypes = [sz, sz, sz, u8p, sz, u8p, f32p, f32p, u32p, u8p, u16p, u8p, i32p]
        L.orc_dequantize_packed.argtypes = [sz, sz, sz, u8p, sz, u8p, u16p, u8p, i32p, C.c_int, C.c_void_p]
        L.orc_bench_inputs.argtypes = [C.c_uint64, sz, sz, sz, sz, C.c_float, f32p, f32p, f32p, C.c_void_p,
                                       C.c_void_p]
        L.orc_rel_err.argtypes = [f32p, f32p, f32p, f32p, sz, sz, sz]
        L.orc_rel_err.restype = C.c_double
        L.orc_rng_new.argtypes = [C.c_void_p, C.c_uint64]
        L.orc_rng_next_u64.argtypes = [C.c_void_p]
        L.orc_rng_next_u64.restype = C.c_uint64
        L.orc_rng_uniform.argtypes = [C.c_void_p]
        L.orc_rng_uniform.restype = C.c_float
        L.orc_rng_normal.argtypes = [C.c_void_p]
        L.orc_rng_normal.restype = C.c_float
        L.orc_synth_normal_at.argtypes = [C.c_uint64, C.c_uint64]
        L.orc_synth_normal_at.restype = C.c_float
        L.orc_synth_normal.argtypes = [C.c_uint64, C.c_uint64, sz, C.c_float, f32p]
        L.orc_synth_outlier_scales.argtypes = [C.c_uint64, sz, C.c_double, C.c_float, f32p]
        L.orc_synth_lognormal_scales.argtypes = [C.c_uint64, sz, C.c_float, f32p]
        L.orc_synth_tokens.argtypes = [C.c_uint64, C.c_uint64, sz, sz, C.c_void_p, f32p]
        L.orc_synth_tokens_heavy.argtypes = [C.c_uint64, C.c_uint64, sz, sz, C.c_void_p, C.c_void_p, f32p]
        L.orc_last_midpoint_counts.argtypes = [C.c_void_p]
        L.orc_set_midpoint_map.argtypes = [C.c_void_p]
        L.orc_synth_student3_at.argtypes = [C.c_uint64, C.c_uint64]
        L.orc_synth_student3_at.restype = C.c_float
        L.orc_synth_log.argtypes = [C.c_double]
        L.orc_synth_log.restype = C.c_double
        L.orc_synth_cos2pi.argtypes = [C.c_double]
        L.orc_synth_cos2pi.restype = C.c_double
        L.orc_set_mutation.argtypes = [C.c_int]
        L.orc_set_threads.argtypes = [C.c_int]
        _lib = L
    return _lib


def config(**kw) -> OrcConfig:
    """A config with the reference defaults (src/engine.rs:146-167), fields overridden by kw.
    `method` accepts "gptq"/"cdcl" or 0/1."""
    c = OrcConfig()
    lib().orc_default_config(C.byref(c))
    for k, v in kw.items():
        if k == "method" and isinstance(v, str):
            v = {"gptq": 0, "cdcl": 1}[v.lower()]
        if isinstance(v, bool):
            v = int(v)
        setattr(c, k, v)
    return c


@dataclass
class QLayer:
    """quant::QLayer (src/quant.rs:161-175) plus the layer stats."""

    d_out: int
    d_in: int
    group: int
    perm: np.ndarray
    gbits: np.ndarray
    codes: np.ndarray
    scales: np.ndarray
    zeros: np.ndarray
    stats: dict

    def dequantize(self) -> np.ndarray:
        out = np.zeros((self.d_out, self.d_in), np.float32)
        lib().orc_dequantize(self.d_out, self.d_in, self.group, self.perm, self.gbits.size, self.codes, self.scales,
                             self.zeros, out)
        return out


class OracleError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


class Cache:
    """One-entry PrepCache (src/engine.rs:220-223)."""

    def __init__(self):
        self.ptr = lib().orc_cache_new()

    def __del__(self):
        if getattr(self, "ptr", None) and _lib is not None:
            _lib.orc_cache_free(self.ptr)
            self.ptr = None


def effective_group(cfg: OrcConfig, n: int) -> int:
    return n if (cfg.group == 0 or cfg.group >= n) else int(cfg.group)


def quantize_layer(w, h, cfg: OrcConfig, m=None, hkey="layer", cache: Cache | None = None, nthreads: int = 8,
                   midmap: bool = False) -> QLayer:
    """engine::quantize_layer (src/engine.rs:690-799) on the CPU oracle. The result's `midpoint`
    holds the near-midpoint accounting; with midmap=True, `midmap` the per-element map (bit 0
    phase-1 code, bit 1 descent, bit 2 zero point)."""
    w = np.ascontiguousarray(w, np.float32)
    h = np.ascontiguousarray(h, np.float32)
    d_out, n = w.shape
    assert h.shape == (n, n)
    if m is not None:
        m = np.ascontiguousarray(m, np.float32)
        assert m.shape == (n, n)
    cache = cache or Cache()
    g = effective_group(cfg, n)
    ng = (n + g - 1) // g
    codes = np.zeros((d_out, n), np.uint8)
    scales = np.zeros((d_out, ng), np.float32)
    zeros = np.zeros((d_out, ng), np.float32)
    perm = np.zeros(n, np.uint32)
    gbits = np.zeros(ng, np.uint8)
    st = OrcStats()
    err = C.create_string_buffer(512)
    mmap = np.zeros((d_out, n), np.uint8) if midmap else None
    lib().orc_set_midpoint_map(mmap.ctypes.data if midmap else None)
    try:
        rc = lib().orc_quantize_layer(w, d_out, n, h, m.ctypes.data if m is not None else None, hkey.encode(),
                                      C.byref(cfg), nthreads, cache.ptr, codes, scales, zeros, perm, gbits, C.byref(st),
                                      err, 512)
    finally:
        lib().orc_set_midpoint_map(None)
    if rc != 0:
        raise OracleError(rc, err.value.decode())
    q = QLayer(d_out, n, g, perm, gbits, codes, scales, zeros, st.as_dict())
    mc = (C.c_uint64 * 6)()
    lib().orc_last_midpoint_counts(mc)
    q.midpoint = dict(zip(MIDPOINT_FIELDS, (int(v) for v in mc)))
    q.midmap = mmap
    return q


MIDPOINT_FIELDS = ("code_decisions", "code_near", "zero_decisions", "zero_near", "cd_decisions", "cd_near")


def gram_accumulate(x, y=None, h=None) -> np.ndarray:
    """linalg::gram_accumulate (src/linalg.rs:388-418): h += x^T y in f64."""
    x = np.ascontiguousarray(x, np.float32)
    y = x if y is None else np.ascontiguousarray(y, np.float32)
    t, n = x.shape
    assert y.shape == (t, n)
    if h is None:
        h = np.zeros((n, n), np.float64)
    lib().orc_gram_accumulate(x, y, t, n, h)
    return h


def upper_chol_of_inverse(h64) -> np.ndarray:
    """linalg::upper_chol_of_inverse (src/linalg.rs:362-375)."""
    h64 = np.ascontiguousarray(h64, np.float64)
    n = h64.shape[0]
    u = np.zeros((n, n), np.float32)
    err = C.create_string_buffer(512)
    rc = lib().orc_upper_chol_of_inverse(h64, n, u, err, 512)
    if rc != 0:
        raise OracleError(rc, err.value.decode())
    return u


def cholesky_lower(a64) -> np.ndarray:
    a = np.array(a64, np.float64, order="C", copy=True)
    err = C.create_string_buffer(512)
    rc = lib().orc_cholesky_lower(a, a.shape[0], err, 512)
    if rc != 0:
        raise OracleError(rc, err.value.decode())
    return a


def tri_inverse_lower(l64) -> np.ndarray:
    l64 = np.ascontiguousarray(l64, np.float64)
    y = np.zeros_like(l64)
    lib().orc_tri_inverse_lower(l64, l64.shape[0], y)
    return y


def sgemm(a, b, c=None, alpha=1.0, beta=0.0) -> np.ndarray:
    """C = alpha*A*B + beta*C with the matrixmultiply chain order (row-major operands)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.zeros((m, n), np.float32) if c is None else np.array(c, np.float32, order="C", copy=True)
    lib().orc_sgemm(m, k, n, alpha, a.ctypes.data, k, 1, b.ctypes.data, n, 1, beta, c.ctypes.data, n, 1)
    return c


def dgemm(a, b, c=None, alpha=1.0, beta=0.0) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float64)
    b = np.ascontiguousarray(b, np.float64)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.zeros((m, n), np.float64) if c is None else np.array(c, np.float64, order="C", copy=True)
    lib().orc_dgemm(m, k, n, alpha, a.ctypes.data, k, 1, b.ctypes.data, n, 1, beta, c.ctypes.data, n, 1)
    return c


def proxy_loss(w_t, w_hat, h) -> float:
    w_t = np.ascontiguousarray(w_t, np.float32)
    w_hat = np.ascontiguousarray(w_hat, np.float32)
    h = np.ascontiguousarray(h, np.float32)
    return lib().orc_proxy_loss(w_t, w_hat, w_t.shape[0], w_t.shape[1], h)


def rtn_layer(w, cfg: OrcConfig) -> np.ndarray:
    w = np.ascontiguousarray(w, np.float32)
    out = np.zeros_like(w)
    lib().orc_rtn_layer(w, w.shape[0], w.shape[1], C.byref(cfg), out)
    return out


def find_params(vals, bits, mse=False):
    vals = np.ascontiguousarray(vals, np.float32)
    s, z = C.c_float(), C.c_float()
    lib().orc_find_params(vals, vals.size, bits, int(mse), C.byref(s), C.byref(z))
    return s.value, z.value


def quant_code(x, scale, zero, maxq):
    c = C.c_uint8()
    dq = lib().orc_quant_code(x, scale, zero, maxq, C.byref(c))
    return c.value, dq


def round_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_round_f16_array(x.ravel(), y.ravel(), x.size)
    return y


# ---------------------------------------------------------------- packed container (cdclq-v1)
DTYPES = {"F32": 0, "F16": 1, "BF16": 2}
_NP_OUT = {0: np.float32, 1: np.uint16, 2: np.uint16}


def row_bytes(n: int, g: int, gbits) -> int:
    """quant::row_bytes (src/quant.rs:102-104)."""
    gbits = np.ascontiguousarray(gbits, np.uint8)
    return lib().orc_row_bytes(n, g, gbits)


def pack_row(codes, g: int, gbits) -> np.ndarray:
    """quant::pack_row (src/quant.rs:113-131)."""
    codes = np.ascontiguousarray(codes, np.uint8)
    gbits = np.ascontiguousarray(gbits, np.uint8)
    out = np.zeros(row_bytes(codes.size, g, gbits), np.uint8)
    lib().orc_pack_row(codes, codes.size, g, gbits, out)
    return out


def unpack_row(data, n: int, g: int, gbits) -> np.ndarray:
    """quant::unpack_row (src/quant.rs:136-151)."""
    data = np.ascontiguousarray(data, np.uint8)
    gbits = np.ascontiguousarray(gbits, np.uint8)
    codes = np.zeros(n, np.uint8)
    lib().orc_unpack_row(data, n, g, gbits, codes)
    return codes


def pack_layer(codes, scales, zeros, perm, gbits, g: int):
    """io::packed_tensors (src/io.rs:244-264): (qweight, scales f16 bits, qzeros, perm i32)."""
    codes = np.ascontiguousarray(codes, np.uint8)
    d_out, n = codes.shape
    gbits = np.ascontiguousarray(gbits, np.uint8)
    ng = gbits.size
    rb = row_bytes(n, g, gbits)
    qw = np.zeros((d_out, rb), np.uint8)
    s16 = np.zeros((d_out, ng), np.uint16)
    qz = np.zeros((d_out, ng), np.uint8)
    p32 = np.zeros(n, np.int32)
    lib().orc_pack_layer(d_out, n, g, gbits, ng, codes, np.ascontiguousarray(scales, np.float32),
                         np.ascontiguousarray(zeros, np.float32), np.ascontiguousarray(perm, np.uint32), qw, s16, qz,
                         p32)
    return qw, s16, qz, p32


def dequantize_packed(qweight, scales16, qzeros, perm32, gbits, g: int, dtype: str = "F32") -> np.ndarray:
    """io::read_packed_layer + QLayer::dequantize + io::f32_to_bytes (src/io.rs:270-293,
    src/quant.rs:189-236, src/io.rs:50-57). F16/BF16 results are returned as uint16 bit patterns."""
    qweight = np.ascontiguousarray(qweight, np.uint8)
    gbits = np.ascontiguousarray(gbits, np.uint8)
    perm32 = np.ascontiguousarray(perm32, np.int32)
    d_out, n = qweight.shape[0], perm32.size
    dt = DTYPES[dtype]
    out = np.zeros((d_out, n), _NP_OUT[dt])
    lib().orc_dequantize_packed(d_out, n, g, gbits, gbits.size, qweight, np.ascontiguousarray(scales16, np.uint16),
                                np.ascontiguousarray(qzeros, np.uint8), perm32, dt, out.ctypes.data)
    return out


def narrow(v, dtype: str) -> np.ndarray:
    """io::f32_to_bytes (src/io.rs:50-57); F16/BF16 as uint16 bit patterns."""
    v = np.ascontiguousarray(v, np.float32)
    dt = DTYPES[dtype]
    out = np.zeros(v.shape, _NP_OUT[dt])
    lib().orc_narrow(v.ravel(), v.size, dt, out.ctypes.data)
    return out


# ---------------------------------------------------------------- synthetic benchmark (src/bench.rs)
def bench_inputs(seed: int, rows: int, n: int, tokens: int, test_tokens: int, asym_noise: float = 0.0):
    """(w, x, xte, xt, xte_t) of bench::run (src/bench.rs:41-97, :275-295); xt/xte_t None without noise."""
    w = np.zeros((rows, n), np.float32)
    x = np.zeros((tokens, n), np.float32)
    xte = np.zeros((test_tokens, n), np.float32)
    xt = xte_t = None
    if asym_noise > 0:
        xt = np.zeros((tokens, n), np.float32)
        xte_t = np.zeros((test_tokens, n), np.float32)
    lib().orc_bench_inputs(seed, rows, n, tokens, test_tokens, asym_noise, w, x, xte,
                           xt.ctypes.data if xt is not None else None, xte_t.ctypes.data if xte_t is not None else None)
    return w, x, xte, xt, xte_t


def rel_err(w, wq, x, xt, rows: int, n: int, t: int) -> float:
    """bench::rel_err (src/bench.rs:106-121)."""
    f = lambda a: np.ascontiguousarray(a, np.float32)
    return lib().orc_rel_err(f(w), f(wq), f(x), f(xt), rows, n, t)


class Rng:
    """rng::Rng (src/rng.rs)."""

    class _S(C.Structure):
        _fields_ = [("s", C.c_uint64), ("has_spare", C.c_int32), ("spare", C.c_float)]

    def __init__(self, seed: int):
        self.st = Rng._S()
        lib().orc_rng_new(C.byref(self.st), seed)

    def next_u64(self) -> int:
        return lib().orc_rng_next_u64(C.byref(self.st))

    def uniform(self) -> float:
        return lib().orc_rng_uniform(C.byref(self.st))

    def normal(self) -> float:
        return lib().orc_rng_normal(C.byref(self.st))


# ---------------------------------------------------------------- synthetic inputs
def synth_normal(seed: int, n: int, sigma: float = 1.0, offset: int = 0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_synth_normal(seed, offset, n, sigma, out)
    return out


def synth_outlier_scales(seed: int, n: int, frac: float, factor: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_synth_outlier_scales(seed, n, frac, factor, out)
    return out


def synth_lognormal_scales(seed: int, n: int, sigma: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_synth_lognormal_scales(seed, n, sigma, out)
    return out


def synth_tokens(seed: int, t: int, n: int, ch_scale=None, row0: int = 0, heavy=None) -> np.ndarray:
    """Token-major t x n inputs; `heavy` (n bools, optional) marks Student-t(3) channels."""
    x = np.empty((t, n), np.float32)
    cs = hv = None
    if ch_scale is not None:
        ch_scale = np.ascontiguousarray(ch_scale, np.float32)
        cs = ch_scale.ctypes.data
    if heavy is not None:
        heavy = np.ascontiguousarray(heavy, np.uint8)
        hv = heavy.ctypes.data
    lib().orc_synth_tokens_heavy(seed, row0, t, n, cs, hv, x)
    return x


def set_threads(n: int):
    lib().orc_set_threads(n)


class mutation:
    """Context manager planting a known mistake in the oracle (tests of the pinning checks)."""

    def __init__(self, mid: int):
        self.mid = mid

    def __enter__(self):
        lib().orc_set_mutation(self.mid)
        return self

    def __exit__(self, *a):
        lib().orc_set_mutation(0)

"""Shared test inputs: the reference's engine-test generator, counter-based synthetic layers and
the reference's Hessian fixtures (copied under tests/golden/)."""
from __future__ import annotations

import ctypes as C
import glob
import os

import numpy as np

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

_libm = C.CDLL("libm.so.6")
_libm.expf.restype = C.c_float
_libm.expf.argtypes = [C.c_float]


def _normals(r: O.Rng, k: int) -> np.ndarray:
    return np.array([r.normal() for _ in range(k)], np.float32)


def ref_problem(d_out: int, n: int, tokens: int, seed: int):
    """src/engine.rs:850-869: low-rank (n/4) correlated activations with log-normal channel scales,
    additive noise, W ~ 0.05 N(0,1); H = gram_accumulate(x, x) cast to f32. Same draw order."""
    r = O.Rng(seed)
    rank = n // 4
    sq = np.float32(np.sqrt(np.float32(rank)))
    a = (_normals(r, rank * n) / sq).astype(np.float32).reshape(rank, n)
    z = _normals(r, tokens * rank).reshape(tokens, rank)
    x = O.sgemm(z, a)
    s = np.array([_libm.expf(float(np.float32(0.5) * np.float32(r.normal()))) for _ in range(n)], np.float32)
    noise = _normals(r, tokens * n).reshape(tokens, n)
    x = ((x + np.float32(0.3) * noise) * s[None, :]).astype(np.float32)
    w = (_normals(r, d_out * n) * np.float32(0.05)).astype(np.float32).reshape(d_out, n)
    h = O.gram_accumulate(x).astype(np.float32)
    return w, h


def damped(h: np.ndarray, damp: float) -> np.ndarray:
    """src/engine.rs:873-880."""
    n = h.shape[0]
    mean = 0.0
    for i in range(n):
        mean += float(h[i, i])
    mean /= n
    d = h.copy()
    d[np.arange(n), np.arange(n)] += np.float32(damp * mean)
    return d


def synth_layer(seed: int, d_out: int, n: int, tokens: int, outlier_frac: float = 0.01, outlier_factor: float = 20.0,
                wsigma: float = 0.02):
    """Counter-based synthetic layer (W ~ N(0, wsigma^2); X ~ N(0,1) with round(frac*n) channels
    scaled by `factor`; H = X^T X in f64 then f32), identical to the device generator."""
    cs = O.synth_outlier_scales(seed * 7 + 1, n, outlier_frac, outlier_factor)
    x = O.synth_tokens(seed * 7 + 2, tokens, n, cs)
    w = O.synth_normal(seed * 7 + 3, d_out * n, wsigma).reshape(d_out, n)
    h64 = O.gram_accumulate(x)
    return w, x, h64.astype(np.float32), cs


def fixture_hessians() -> dict:
    """The reference's test fixtures (tests/fixtures/*/hess.safetensors), read with safetensors."""
    from safetensors.numpy import load_file

    out = {}
    for p in sorted(glob.glob(os.path.join(GOLDEN, "hess_*.safetensors"))):
        tag = os.path.basename(p)[len("hess_"):-len(".safetensors")]
        for k, v in load_file(p).items():
            out[f"{tag}:{k}"] = np.ascontiguousarray(v, np.float32)
    return out


def rand_spd(n: int, seed: int) -> np.ndarray:
    """src/linalg.rs:426-443: M M^T + I with M n x (n+8) from rng.normal() (f64 product)."""
    r = O.Rng(seed)
    m = np.array([r.normal() for _ in range(n * (n + 8))], np.float64).reshape(n, n + 8)
    h = m @ m.T
    h[np.arange(n), np.arange(n)] += 1.0
    return h


def gemm_order_failures() -> list:
    """Closed forms that fix matrixmultiply 0.3.8's per-element order (src/linalg.rs:3-6, :93,
    :98-99): each KC = 256 panel is a chain of fused multiply-adds started from 0, folded into C in
    panel order. Each case has an exact answer under that order and a different one under a
    plausible alternative (products rounded before the add, the panel chain started from C, another
    panel width). Returns the names of the cases that fail (empty when the order holds)."""
    bad = []
    # f32: (1 + 2^-12)^2 - 1 = 2^-11 + 2^-24 exactly; a rounded product loses the 2^-24 (a tie
    # between 1 + 2^-11 and its upper neighbour, resolved to the even 1 + 2^-11).
    e = 2.0 ** -12
    a = np.array([[1.0, 1.0 + e]], np.float32)
    b = np.array([[-1.0], [1.0 + e]], np.float32)
    want = 2.0 ** -11 + 2.0 ** -24
    if O.sgemm(a, b)[0, 0] != np.float32(want):
        bad.append("sgemm fused chain")
    if O.sgemm(a, b, alpha=-1.0)[0, 0] != np.float32(-want):
        bad.append("sgemm fused chain, alpha -1")
    c = np.full((1, 1), 2.0 ** -10, np.float32)
    if O.sgemm(a, b, c, alpha=1.0, beta=1.0)[0, 0] != np.float32(2.0 ** -10 + want):
        bad.append("sgemm fused chain, beta 1")
    if O.sgemm(a, b, c, alpha=-1.0, beta=1.0)[0, 0] != np.float32(2.0 ** -10 - want):
        bad.append("sgemm fused chain, alpha -1 beta 1")
    # f32: the panel chain starts at 0 and is added to C once: 1 + (2^-24 + 2^-24) = 1 + 2^-23,
    # whereas a chain started from C = 1 stays at 1 (each 1 + 2^-24 ties to the even 1).
    a2 = np.full((1, 2), 2.0 ** -24, np.float32)
    b2 = np.ones((2, 1), np.float32)
    if O.sgemm(a2, b2, np.ones((1, 1), np.float32), beta=1.0)[0, 0] != np.float32(1.0 + 2.0 ** -23):
        bad.append("sgemm chain from zero, beta 1")
    # f64 analogue of the fused chain: (1 + 2^-27)^2 - 1 = 2^-26 + 2^-54; the rounded product is
    # 1 + 2^-26 (2^-54 is a quarter of an ulp of 1).
    e = 2.0 ** -27
    a = np.array([[1.0, 1.0 + e]])
    b = np.array([[-1.0], [1.0 + e]])
    want = 2.0 ** -26 + 2.0 ** -54
    if O.dgemm(a, b)[0, 0] != want:
        bad.append("dgemm fused chain")
    if O.dgemm(a, b, alpha=-1.0)[0, 0] != -want:
        bad.append("dgemm fused chain, alpha -1")
    c = np.full((1, 1), 2.0 ** -25)
    if O.dgemm(a, b, c, alpha=1.0, beta=1.0)[0, 0] != 2.0 ** -25 + want:
        bad.append("dgemm fused chain, beta 1")
    if O.dgemm(a, b, c, alpha=-1.0, beta=1.0)[0, 0] != 2.0 ** -25 - want:
        bad.append("dgemm fused chain, alpha -1 beta 1")
    # f64 panel width: a[0] b[0] = 2^27 * 2^26 = 2^53, after which every +1 inside the panel ties
    # back to 2^53, while each later panel adds its exact count of ones.
    for k in (256, 258, 600, 1024):
        a = np.ones((1, k))
        b = np.ones((k, 1))
        a[0, 0] = 2.0 ** 27
        b[0, 0] = 2.0 ** 26
        full, rem = divmod(k, 256)
        if O.dgemm(a, b)[0, 0] != 2.0 ** 53 + 256.0 * (full - 1) + rem:
            bad.append(f"dgemm KC panels, k {k}")
    # f32 panel width (2^12 * 2^12 = 2^24; same argument with f32 ties)
    for k in (256, 258, 600, 1024):
        a = np.ones((1, k), np.float32)
        a[0, 0] = 4096.0
        full, rem = divmod(k, 256)
        if O.sgemm(a, a.T.copy())[0, 0] != np.float32(2.0 ** 24 + 256.0 * (full - 1) + rem):
            bad.append(f"sgemm KC panels, k {k}")
    return bad


def row_chunk(d_out: int, row_chunk_cfg: int, nthreads: int) -> int:
    """The reference's row-chunk size (src/engine.rs:768-770)."""
    if row_chunk_cfg > 0:
        rc = row_chunk_cfg
    else:
        rc = min(max(-(-d_out // max(nthreads, 1)), 32), 256)
    return max(min(rc, d_out), 1)


def classify_mismatches(got_codes, want_codes, midmap, rc: int) -> dict:
    """Near-midpoint classification of code mismatches (the parity contract's exemption).

    A mismatching element whose oracle decision was near a midpoint (any bit of `midmap`, see
    oracle.quantize_layer) is exempt: there the reference's own rounding input lies within 1e-9 of
    k + 1/2. Other mismatches in a row chunk of `rc` rows that holds an exempt one are cascaded: a
    different code changes that row's later errors and gradients, and the chunk's shared
    convergence decisions reach its other rows. The rest are non-exempt, i.e. real differences.
    Returns counts: mismatches, exempt, cascaded, non_exempt, rows (with a mismatch), exempt_chunks,
    and `chunk_ids`, the sorted indices of the row chunks holding an exempt mismatch."""
    bad = np.asarray(got_codes) != np.asarray(want_codes)
    rows = np.nonzero(bad.any(axis=1))[0]
    ex = bad & (np.asarray(midmap) != 0)
    ex_chunks = set((np.nonzero(ex.any(axis=1))[0] // rc).tolist())
    total, n_ex = int(bad.sum()), int(ex.sum())
    casc = sum(int(bad[r].sum() - ex[r].sum()) for r in rows if r // rc in ex_chunks)
    return dict(mismatches=total, exempt=n_ex, cascaded=casc, non_exempt=total - n_ex - casc, rows=int(len(rows)),
                exempt_chunks=len(ex_chunks), chunk_ids=sorted(ex_chunks))


# Near-midpoint report of the session's parity comparisons: one record per comparison (label, the
# oracle's counts, the GPU's counts, the mismatch classification or None when the codes are equal).
# tests/conftest.py prints the totals at the end of the run.
MIDPOINT_LOG: list = []


def tie_problem(d_out: int = 48, n: int = 256, g: int = 64, seed: int = 5):
    """A layer whose rounding decisions sit exactly on midpoints: every weight is (k + 1/2) 2^-6 and
    every group spans -4.5 2^-6 .. 10.5 2^-6, so with 4 bits the scale is exactly 2^-6 and each
    x / scale (codes) and -lo / scale (zero points) is an f32 tie; H is diagonal, so the phase-1
    compensation and the descent targets leave the weights on the ties. Natural order, g | n."""
    rng = np.random.default_rng(seed)
    w = ((rng.integers(-5, 11, (d_out, n)) + 0.5) * 2.0 ** -6).astype(np.float32)
    for c0 in range(0, n, g):
        w[:, c0] = np.float32(-4.5 * 2.0 ** -6)
        w[:, c0 + 1] = np.float32(10.5 * 2.0 ** -6)
    h = np.diag(rng.uniform(0.5, 2.0, n)).astype(np.float32)
    return w, h

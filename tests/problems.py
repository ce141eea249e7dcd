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

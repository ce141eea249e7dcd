"""Pins for the oracle's linear algebra (src/linalg.rs:56-542)."""
import numpy as np
import pytest

import oracle as O
from problems import gemm_order_failures, rand_spd


def test_cholesky_matches_definition():
    """src/linalg.rs:447-464: L L^T = A to 1e-10 at n = 150 (crosses the NB = 96 block)."""
    n = 150
    h = rand_spd(n, 1)
    l = np.tril(O.cholesky_lower(h))
    err = np.abs(l @ l.T - h) / np.maximum(np.abs(h), 1.0)
    assert err.max() < 1e-10
    assert np.allclose(l, np.linalg.cholesky(h), rtol=1e-9, atol=1e-12)


def test_upper_factor_of_inverse():
    """src/linalg.rs:470-504: U^T U H = I (5e-4), strictly-lower zeros, positive diagonal; and
    U = chol(H^-1)^T from library routines."""
    n = 200
    h = rand_spd(n, 2)
    u = O.upper_chol_of_inverse(h).astype(np.float64)
    assert np.abs(u.T @ u @ h - np.eye(n)).max() < 5e-4
    assert np.all(np.tril(u, -1) == 0) and np.all(np.diag(u) > 0)
    ref = np.linalg.cholesky(np.linalg.inv(h)).T
    assert np.abs(u - ref).max() / np.abs(ref).max() < 1e-6


@pytest.mark.parametrize("n", [1, 7, 96, 97, 300, 400])
def test_tri_inverse(n):
    rng = np.random.default_rng(n)
    l = np.tril(rng.standard_normal((n, n))) + np.eye(n) * (n + 1.0)
    l_garbage = l + np.triu(rng.standard_normal((n, n)), 1)  # upper triangle must be ignored
    y = O.tri_inverse_lower(l_garbage)
    assert np.abs(y @ l - np.eye(n)).max() < 1e-12
    assert np.all(np.triu(y, 1) == 0)


@pytest.mark.parametrize("h,pivot", [
    ([[4.0, 2.0], [2.0, 1.0]], "pivot 1 = 0e0"),
    ([[1.0, 3.0], [3.0, 1.0]], "pivot 1 = -8e0"),
    ([[float("nan"), 0.0], [0.0, 1.0]], "pivot 1 = NaN"),
    ([[1.0, 0.0], [0.0, -0.001]], "pivot 0 = -1e-3"),
    ([[2.0, 0.0], [0.0, -1234.5]], "pivot 0 = -1.2345e3"),
])
def test_not_pd_message(h, pivot):
    """src/linalg.rs:215-219 message with Rust's `{:e}` formatting of the failing pivot (index in
    the flipped matrix)."""
    with pytest.raises(O.OracleError) as e:
        O.upper_chol_of_inverse(np.array(h))
    assert str(e.value) == f"matrix is not positive definite ({pivot}); increase --damp or check the Hessian"


@pytest.mark.parametrize("m,k,n", [(97, 130, 111), (20, 300, 400), (5, 1000, 3), (64, 256, 64), (33, 513, 17)])
def test_sgemm_matches_f64_product(m, k, n):
    rng = np.random.default_rng(m * k + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    bound = 2 * k * np.finfo(np.float32).eps * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)) + 1e-30
    assert np.all(np.abs(O.sgemm(a, b) - ref) <= bound)
    assert np.all(np.abs(O.sgemm(a, b, c0, alpha=-1.0, beta=1.0) - (c0 - ref)) <= bound + 1e-6 * np.abs(c0))


def test_parallel_gemm_matches_serial():
    """src/linalg.rs:510-541 (stronger here: bit-identical across thread counts, since splitting C
    never changes an element's chain)."""
    rng = np.random.default_rng(3)
    for (m, k, n) in ((97, 130, 111), (20, 300, 400), (300, 700, 300)):
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal((k, n)).astype(np.float32)
        O.set_threads(1)
        c1 = O.sgemm(a, b)
        O.set_threads(4)
        c4 = O.sgemm(a, b)
        O.set_threads(8)
        assert np.array_equal(c1, c4)


def test_gemm_panel_structure_closed_form():
    """KC = 256 panels, each a fused chain from 0, folded in panel order. With a[0] = 2^12 and the
    rest 1, the f32 chain 2^24 + 1 + 1 ... stays at 2^24 (ties to even) inside a panel, while each
    later panel contributes its exact count: C = 2^24 + 256 * (number of later panels) + tail."""
    for k in (256, 257, 600, 1024):
        a = np.ones((1, k), np.float32)
        a[0, 0] = 4096.0
        b = a.T.copy()
        full, rem = divmod(k, 256)
        expect = 2.0 ** 24 + 256.0 * (full - 1) + rem
        assert O.sgemm(a, b)[0, 0] == np.float32(expect), k


def test_gemm_order_closed_forms():
    """Fused chains from 0 per KC = 256 panel, folded in order, for sgemm and dgemm (alpha = +-1,
    beta 0 and 1): the matrixmultiply 0.3.8 order that every GEMM call site of the reference relies
    on (src/engine.rs:454,548,560,608; src/linalg.rs:254,310,326,398)."""
    assert gemm_order_failures() == []


@pytest.mark.parametrize("mid,case", [(11, "sgemm fused chain"), (11, "dgemm fused chain"),
                                      (12, "dgemm KC panels, k 256")])
def test_gemm_order_mutations_fail_the_closed_forms(mid, case):
    with O.mutation(mid):
        assert case in gemm_order_failures()


def test_gram_chunks_closed_form():
    """H += (f64) chunk sums over 2048-token chunks (src/linalg.rs:392-417): the f64 accumulator
    keeps what the f32 chunk loses. x[0] = 2^12, the rest 1: chunk 0 gives 2^24 + 7*256, every later
    chunk its exact count."""
    for t in (2047, 2048, 2049, 4097, 6000):
        x = np.ones((t, 1), np.float32)
        x[0, 0] = 4096.0
        h = O.gram_accumulate(x)
        c0 = min(t, 2048)
        p, r = divmod(c0, 256)
        expect = float(np.float32(2.0 ** 24 + 256.0 * (p - 1) + r)) + (t - c0)
        assert h[0, 0] == expect, t


@pytest.mark.parametrize("t,n", [(100, 16), (2049, 33), (5000, 40)])
def test_gram_brute_force_and_symmetry(t, n):
    rng = np.random.default_rng(t)
    x = (rng.standard_normal((t, n)) * rng.uniform(0.1, 30, n)).astype(np.float32)
    y = (x + rng.standard_normal((t, n))).astype(np.float32)
    h = O.gram_accumulate(x)
    assert np.array_equal(h, h.T)  # exact: fma(a, b, c) == fma(b, a, c)
    ref = x.astype(np.float64).T @ x.astype(np.float64)
    scale = np.abs(x).astype(np.float64).T @ np.abs(x).astype(np.float64)
    assert np.all(np.abs(h - ref) <= 2049 * np.finfo(np.float32).eps * scale)
    hm = O.gram_accumulate(x, y)
    refm = x.astype(np.float64).T @ y.astype(np.float64)
    scalem = np.abs(x).astype(np.float64).T @ np.abs(y).astype(np.float64)
    assert np.all(np.abs(hm - refm) <= 2049 * np.finfo(np.float32).eps * scalem)
    h2 = O.gram_accumulate(x, h=np.ones((n, n)))
    assert np.array_equal(h2, O.gram_accumulate(x, h=np.ones((n, n))))

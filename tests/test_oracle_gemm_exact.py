"""The oracle's GEMM against an exact restatement of matrixmultiply 0.3.8's per-element order
(src/linalg.rs:56-184 call it; the crate is a Cargo.lock dependency absent from the reference
tree): for every C element and every KC-wide panel of k in order, acc = fma(a_ik, b_kj, acc) from
+0 in k order, then C = fma(alpha, acc, C') with C' = beta * C for the first panel (0 when beta is
0) and C afterwards. Here every fma is evaluated exactly in rational arithmetic and rounded once
to the target format (ties to even), so the check does not depend on any floating-point unit.

The shapes exercise every path of the oracle's loop nest: 6- and 4-row register blocks and the
scalar rows after them, 16-column (f32) / 8-column (f64) vector blocks and the scalar columns
after them, several KC panels with a ragged last one, transposed (strided) operands, and the
alpha / beta forms the engine uses. Small sizes: the exact chains run in Python."""
from fractions import Fraction

import numpy as np
import pytest

import oracle as O

KC = 256


def _round_f32(x: Fraction) -> np.float32:
    """x rounded once to the nearest f32, ties to even (finite, in range)."""
    d = np.float32(float(x))  # within one f32 step of the answer
    cands = [np.nextafter(d, np.float32(-np.inf)), d, np.nextafter(d, np.float32(np.inf))]
    return min(cands, key=lambda c: (abs(Fraction(float(c)) - x), int(np.array(c).view(np.uint32)) & 1))


def _fma(a, b, c, f32: bool):
    """Exact a*b + c rounded once; an exact zero keeps IEEE's sign rule (-0 only for -0 + -0)."""
    s = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    if s == 0:
        prod_neg = (np.signbit(a) != np.signbit(b)) and (a == 0 or b == 0)
        neg = prod_neg and np.signbit(c) and c == 0
        z = -0.0 if neg else 0.0
        return np.float32(z) if f32 else z
    return _round_f32(s) if f32 else float(s)


def exact_gemm(a, b, c0, alpha, beta, f32: bool):
    m, k = a.shape
    n = b.shape[1]
    out = np.zeros((m, n), np.float32 if f32 else np.float64)
    typ = np.float32 if f32 else np.float64
    zero = typ(0.0)
    for i in range(m):
        for j in range(n):
            c = (zero if beta == 0 else typ(typ(beta) * c0[i, j]))
            for k0 in range(0, k, KC):
                acc = zero
                for kk in range(k0, min(k, k0 + KC)):
                    acc = typ(_fma(a[i, kk], b[kk, j], acc, f32))
                c = typ(_fma(typ(alpha), acc, c, f32))
            out[i, j] = c
    return out


def _operands(rng, m, k, n, dt):
    # varied magnitudes and signs, some exact zeros, products that cancel
    a = (rng.standard_normal((m, k)) * np.exp2(rng.integers(-12, 12, (m, k)))).astype(dt)
    b = (rng.standard_normal((k, n)) * np.exp2(rng.integers(-6, 6, (k, n)))).astype(dt)
    a[rng.random((m, k)) < 0.05] = 0.0
    b[rng.random((k, n)) < 0.05] = -0.0
    c0 = rng.standard_normal((m, n)).astype(dt)
    return a, b, c0


def _oracle(fn, a, b, c0, alpha, beta, ta, tb):
    m, k = a.shape
    n = b.shape[1]
    A = np.ascontiguousarray(a.T) if ta else a
    B = np.ascontiguousarray(b.T) if tb else b
    rsa, csa = (1, m) if ta else (k, 1)
    rsb, csb = (1, k) if tb else (n, 1)
    c = c0.copy()
    fn(m, k, n, alpha, A.ctypes.data, rsa, csa, B.ctypes.data, rsb, csb, beta, c.ctypes.data, n, 1)
    return c


# (m, k, n): 6-row blocks + 4-row block + scalar rows (m = 11, 17), vector and scalar columns
# (n = 19, 37), one row, ragged KC panels (k = 300, 513), k = 1
SHAPES = [(11, 300, 19), (17, 40, 37), (1, 513, 17), (6, 1, 16), (5, 257, 9)]
FORMS = [(1.0, 0.0, False, False), (-1.0, 1.0, True, False), (1.0, 1.0, False, True), (0.5, -0.5, True, True)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("f32", [True, False], ids=["sgemm", "dgemm"])
def test_oracle_gemm_equals_exact_chain(shape, f32):
    rng = np.random.default_rng(hash((shape, f32)) % 2 ** 32)
    m, k, n = shape
    dt = np.float32 if f32 else np.float64
    lib = O.lib()
    fn = lib.orc_sgemm if f32 else lib.orc_dgemm
    a, b, c0 = _operands(rng, m, k, n, dt)
    for alpha, beta, ta, tb in FORMS:
        got = _oracle(fn, a, b, c0, alpha, beta, ta, tb)
        want = exact_gemm(a, b, c0, alpha, beta, f32)
        bits = np.uint32 if f32 else np.uint64
        bad = np.argwhere(got.view(bits) != want.view(bits))
        assert bad.size == 0, (f"{'sgemm' if f32 else 'dgemm'} {shape} alpha {alpha} beta {beta} ta {ta} tb {tb}: "
                               f"{len(bad)} elements differ, first {bad[0].tolist()}: oracle {got[tuple(bad[0])]!r} "
                               f"exact {want[tuple(bad[0])]!r}")


def test_exact_chain_catches_the_unfused_mutation():
    """The planted 'every product rounded' mutation of the oracle differs from the exact chain on
    these operands, so the comparison above can see a wrong per-element order."""
    rng = np.random.default_rng(5)
    a, b, c0 = _operands(rng, 7, 300, 19, np.float32)
    want = exact_gemm(a, b, c0, 1.0, 0.0, True)
    with O.mutation(11):
        got = _oracle(O.lib().orc_sgemm, a, b, c0, 1.0, 0.0, False, False)
    assert not np.array_equal(got.view(np.uint32), want.view(np.uint32))

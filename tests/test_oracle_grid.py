"""Pins for the oracle's grid arithmetic (src/quant.rs:20-95) and rng (src/rng.rs)."""
import numpy as np
import pytest

import oracle as O

F16_MIN = np.float32(2.0 ** -14)


def _check_f16(bits):
    x = bits.view(np.float32)
    got = O.round_f16(x)
    with np.errstate(over="ignore", invalid="ignore"):
        exp = x.astype(np.float16).astype(np.float32)
    nan = np.isnan(x)
    assert np.array_equal(np.isnan(got), nan)
    ok = got.view(np.uint32)[~nan] == exp.view(np.uint32)[~nan]
    assert ok.all(), f"first mismatch at bits {bits[~nan][~ok][0]:#x}"


def test_round_f16_vs_ieee_binary16():
    """round_f16 == IEEE binary16 round-to-nearest-even (numpy's float16 conversion is an
    independent RNE implementation). Exhaustive over every f32 whose f16 result is normal
    (exponents 113..142, both signs, all mantissas: every tie and carry case); stride 11 (which
    visits every residue of the 13 rounded-off bits) over the subnormal-result and overflow
    bands; a coarse stride over the rest (zeros, tiny values, inf, NaN)."""
    for sign in (0, 1 << 31):
        for e in range(113, 143):
            base = sign | (e << 23)
            _check_f16(np.arange(base, base + (1 << 23), dtype=np.uint64).astype(np.uint32))
        for lo, hi in ((100, 113), (143, 151)):
            base = sign | (lo << 23)
            _check_f16(np.arange(base, sign | (hi << 23), 11, dtype=np.uint64).astype(np.uint32))
    _check_f16(np.arange(0, 1 << 32, 65537, dtype=np.uint64).astype(np.uint32))
    special = np.array([0x0, 0x80000000, 0x7F800000, 0xFF800000, 0x477FF000, 0x477FEFFF, 0x477FF001, 0x33000000,
                        0x33000001, 0x32FFFFFF, 0x387FC000, 0x387FE000], np.uint32)
    _check_f16(special)


def test_grid_reproduces_zero_and_is_f16_exact():
    """src/quant.rs:279-286."""
    v = ((np.arange(64, dtype=np.float32) - np.float32(20.0)) * np.float32(0.013)).astype(np.float32)
    s, z = O.find_params(v, 3, False)
    assert np.float32(s) == O.round_f16(np.array([s], np.float32))[0]
    _, d0 = O.quant_code(0.0, s, z, 7.0)
    assert abs(d0) < 1e-6


def _rround(t):
    """Rust f32::round: half away from zero (exact in f64 for any f32 input)."""
    t = float(np.float32(t))
    return np.float32(np.copysign(np.floor(abs(t) + 0.5), t))


def _find_params_closed_form(vals, bits):
    """P1: range containing 0, all-zero -> [-1, 1], f16 scale floored at 2^-14, integer zero."""
    maxq = np.float32((1 << bits) - 1)
    lo = min(np.float32(0), vals.min())
    hi = max(np.float32(0), vals.max())
    if lo == 0 and hi == 0:
        lo, hi = np.float32(-1), np.float32(1)
    s = np.float32(np.float16(np.float32(hi - lo) / maxq))
    s = max(s, F16_MIN)
    z = np.float32(min(max(_rround(np.float32(-lo) / s), np.float32(0)), maxq))
    return s, z


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_find_params_minmax_closed_form(bits):
    rng = np.random.default_rng(bits)
    for trial in range(300):
        n = int(rng.integers(1, 200))
        scale = 10.0 ** rng.uniform(-7, 2)
        vals = (rng.standard_normal(n) * scale).astype(np.float32)
        if trial % 10 == 0:
            vals = np.abs(vals)  # range must still contain 0
        if trial % 37 == 0:
            vals[:] = 0  # all-zero group
        s, z = O.find_params(vals, bits, False)
        es, ez = _find_params_closed_form(vals, bits)
        assert np.float32(s).view(np.uint32) == es.view(np.uint32), (trial, s, es)
        assert z == ez
        assert s >= F16_MIN and 0 <= z <= (1 << bits) - 1


def _quant(x, s, z, maxq):
    """P2 with Rust's round (half away from zero)."""
    r = _rround(np.float32(x) / np.float32(s))
    q = np.float32(min(max(np.float32(r + z), np.float32(0)), maxq))
    return int(q), np.float32(s * np.float32(q - z))


def test_quant_code_round_half_away_and_saturation():
    s, z, maxq = np.float32(0.5), np.float32(3), np.float32(7)
    # exact ties round away from zero: 0.25/0.5 = 0.5 -> 1, -0.25/0.5 = -0.5 -> -1
    assert O.quant_code(0.25, s, z, maxq)[0] == 4
    assert O.quant_code(-0.25, s, z, maxq)[0] == 2
    assert O.quant_code(100.0, s, z, maxq)[0] == 7  # saturates high
    assert O.quant_code(-100.0, s, z, maxq)[0] == 0  # saturates low
    rng = np.random.default_rng(1)
    for _ in range(2000):
        bits = int(rng.integers(2, 9))
        maxq = np.float32((1 << bits) - 1)
        s = np.float32(np.float16(rng.uniform(1e-4, 1)))
        z = np.float32(rng.integers(0, int(maxq) + 1))
        x = np.float32(rng.standard_normal() * float(s) * float(maxq) / 2)
        c, dq = O.quant_code(float(x), float(s), float(z), float(maxq))
        ec, edq = _quant(x, s, z, maxq)
        assert c == ec and np.float32(dq) == edq


@pytest.mark.parametrize("bits", [2, 3])
def test_find_params_mse_brute_force(bits):
    """P1 clip search: 24 ratios p = 1 - 0.02 i, sequential f32 squared-error sum, first strict
    minimum wins (brute force in numpy scalars)."""
    rng = np.random.default_rng(10 + bits)
    maxq = np.float32((1 << bits) - 1)
    for trial in range(40):
        vals = (rng.standard_normal(64) * 0.02).astype(np.float32)
        vals[int(rng.integers(0, 64))] *= np.float32(6)  # an outlier worth clipping
        xmin, xmax = min(np.float32(0), vals.min()), max(np.float32(0), vals.max())
        best, best_err = None, np.float32(np.inf)
        for i in range(24):
            p = np.float32(np.float32(1) - np.float32(0.02) * np.float32(i))
            lo, hi = np.float32(p * xmin), np.float32(p * xmax)
            s = max(np.float32(np.float16(np.float32(hi - lo) / maxq)), F16_MIN)
            z = np.float32(min(max(_rround(np.float32(-lo) / s), np.float32(0)), maxq))
            err = np.float32(0)
            for v in vals:
                _, d = _quant(v, s, z, maxq)
                e = np.float32(d - v)
                err = np.float32(err + np.float32(e * e))
            if err < best_err:
                best_err, best = err, (s, z)
        s, z = O.find_params(vals, bits, True)
        assert (np.float32(s), np.float32(z)) == best, trial


def test_splitmix64_known_answers():
    """Rng::new(seed) starts at seed + gamma and adds gamma before mixing (src/rng.rs:22-34), so
    seed = -gamma mod 2^64 reproduces the published splitmix64 sequence for state 0."""
    g = 0x9E3779B97F4A7C15
    r = O.Rng((-g) % (1 << 64))
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC, 0x1B39896A51A8749B]
    assert [r.next_u64() for _ in range(5)] == want


def test_rng_uniform_and_normal_shape():
    r = O.Rng(7)
    u = np.array([r.uniform() for _ in range(20000)])
    assert u.min() > 0 and u.max() < 1 and abs(u.mean() - 0.5) < 0.01
    r = O.Rng(7)
    k = r.next_u64()
    r2 = O.Rng(7)
    assert r2.uniform() == np.float32(((k >> 40) + 0.5) / (1 << 24))
    z = np.array([O.Rng(s).normal() for s in range(4000)])
    assert abs(z.mean()) < 0.06 and abs(z.std() - 1) < 0.05


def test_synth_normal_distribution_and_determinism():
    z = O.synth_normal(3, 1 << 18)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    assert abs((z ** 3).mean()) < 0.03 and abs((z ** 4).mean() - 3) < 0.05
    assert np.array_equal(z[1000:2000], O.synth_normal(3, 1000, offset=1000))
    x = np.linspace(1e-12, 1, 5001)
    assert np.abs(np.array([O.lib().orc_synth_log(v) for v in x]) - np.log(x)).max() < 1e-13
    assert np.abs(np.array([O.lib().orc_synth_cos2pi(v) for v in x]) - np.cos(2 * np.pi * x)).max() < 1e-13
    cs = O.synth_outlier_scales(1, 2048, 0.01, 20.0)
    assert (cs == 20.0).sum() == 20 and (cs == 1.0).sum() == 2028

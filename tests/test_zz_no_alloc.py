"""The allocation-free Gram entry point (cdclq_gram_accumulate_device_noalloc) against the
allocating one (cdclq_gram_accumulate_device), through the C ABI: bit-identical H on two calls in
a row, the second with a smaller input (the fixed scratch keeps the first call's contents), for the
symmetric and the cross-covariance paths, plus the size limit."""
import ctypes as C

import numpy as np
import pytest

import cdclq

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = cdclq.Context(0)
    yield c
    c.close()


def _pair(ctx, x, y, h0, noalloc):
    t, n = x.shape
    dx = cdclq.DeviceArray.from_host(ctx, x)
    dy = dx if y is x else cdclq.DeviceArray.from_host(ctx, y)
    dh = cdclq.DeviceArray.from_host(ctx, h0)
    fn = cdclq.lib().cdclq_gram_accumulate_device_noalloc if noalloc else cdclq.lib().cdclq_gram_accumulate_device
    ctx.check(fn(ctx.ptr, dx.ptr, dy.ptr, t, n, dh.ptr))
    out = dh.download()
    for d in {id(a): a for a in (dx, dy, dh)}.values():
        d.free()
    return out


@pytest.mark.parametrize("sym", [True, False])
def test_noalloc_gram_matches_allocating_entry_point(ctx, sym):
    rng = np.random.default_rng(17 if sym else 18)
    # first call larger (direct-to-LDS tiles, n % 128 == 0), second smaller and ragged (n % 128 != 0)
    for (t, n) in ((4160, 1024), (2100, 200)):
        x = (rng.standard_normal((t, n)) * rng.uniform(0.1, 8, n)).astype(np.float32)
        y = x if sym else (x + 0.05 * rng.standard_normal((t, n))).astype(np.float32)
        h0 = np.zeros((n, n)) if sym else rng.standard_normal((n, n))
        print(f"[noalloc] sym={sym} t={t} n={n}", flush=True)
        want = _pair(ctx, x, y, h0, noalloc=False)
        got = _pair(ctx, x, y, h0, noalloc=True)
        assert np.array_equal(got.view(np.uint64), want.view(np.uint64)), (sym, t, n)


def test_noalloc_gram_symmetric_start_not_bitwise_symmetric(ctx):
    """A symmetric call onto an H that is not bitwise symmetric takes the unmirrored tile list (the
    status word in the fixed scratch must be cleared by each call, not left from the last one)."""
    rng = np.random.default_rng(19)
    t, n = 2048, 256
    x = rng.standard_normal((t, n)).astype(np.float32)
    _pair(ctx, x, x, np.zeros((n, n)), noalloc=True)  # leaves status 0
    h0 = rng.standard_normal((n, n))
    assert np.array_equal(_pair(ctx, x, x, h0, noalloc=True).view(np.uint64),
                          _pair(ctx, x, x, h0, noalloc=False).view(np.uint64))
    _pair(ctx, x, x, h0, noalloc=True)  # leaves status 1
    hs = np.zeros((n, n))
    assert np.array_equal(_pair(ctx, x, x, hs, noalloc=True).view(np.uint64),
                          _pair(ctx, x, x, hs, noalloc=False).view(np.uint64))


def test_noalloc_gram_rejects_n_above_the_limit(ctx):
    """n = 32769 exceeds the fixed scratch: an error before any device work (the pointers are never
    dereferenced, so small dummy buffers serve)."""
    d = cdclq.DeviceArray(ctx, 64, np.float64)
    rc = cdclq.lib().cdclq_gram_accumulate_device_noalloc(ctx.ptr, d.ptr, d.ptr, 1, 32769, d.ptr)
    assert rc == cdclq.INVALID_ARG
    assert "exceeds the allocation-free limit of 32768" in cdclq.lib().cdclq_last_error(ctx.ptr).decode()
    d.free()


def _free_bytes():
    hip = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(0), C.c_size_t(0)
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def test_noalloc_gram_leaves_device_memory_unchanged():
    """On a context that has never grown its workspace, the allocation-free call leaves the
    device's free memory exactly as it was (inputs allocated beforehand, output read after the
    second probe); the allocating call on another fresh context is printed as the contrast."""
    rng = np.random.default_rng(23)
    t, n = 4096, 512
    x = rng.standard_normal((t, n)).astype(np.float32)
    warm = cdclq.Context(0)
    _pair(warm, x, x, np.zeros((n, n)), noalloc=True)  # code objects and the fixed array in place
    warm.close()
    for noalloc in (True, False):
        c = cdclq.Context(0)
        dx = cdclq.DeviceArray.from_host(c, x)
        dh = cdclq.DeviceArray.from_host(c, np.zeros((n, n)))
        fn = cdclq.lib().cdclq_gram_accumulate_device_noalloc if noalloc else cdclq.lib().cdclq_gram_accumulate_device
        before = _free_bytes()
        c.check(fn(c.ptr, dx.ptr, dx.ptr, t, n, dh.ptr))
        after = _free_bytes()
        print(f"[noalloc] noalloc={noalloc}: free device memory {before} -> {after}", flush=True)
        if noalloc:
            assert after == before, f"the allocation-free call changed free device memory by {after - before}"
        for d in (dx, dh):
            d.free()
        c.close()

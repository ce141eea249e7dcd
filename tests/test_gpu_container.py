"""GPU parity of the packed container cdclq-v1 (src/quant.rs:98-236, src/io.rs:50-57, :244-293):
the HIP pack / dequantize kernels through the C ABI against the CPU oracle on identical inputs.

Bar: every output byte identical (qweight, f16 scale bits, u8 zero points, i32 perm, and the
dequantized F32 / F16 / BF16 tensors bit for bit). NaN results of the dequantization (a NaN or
infinite scale meeting code == zero) carry a platform-defined payload and sign in the reference
(x86 gives the default NaN); those are compared as "both NaN" only.
"""
import numpy as np
import pytest

import cdclq
import oracle as O
from problems import synth_layer

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = cdclq.Context(0)
    yield c
    c.close()


def _layer(n, g, d_out, seed, wild=False, specials=False, gb=None, act_order=True):
    rng = np.random.default_rng(seed)
    ng = (n + g - 1) // g
    gbits = (np.asarray(gb, np.uint8) if gb is not None else rng.integers(1, 9, ng).astype(np.uint8))
    w = gbits.astype(np.int64)[np.arange(n) // g]
    codes = rng.integers(0, 256, (d_out, n))
    if not wild:
        codes &= (1 << w) - 1
    codes = codes.astype(np.uint8)
    scales = O.round_f16(rng.uniform(1e-4, 0.3, (d_out, ng)).astype(np.float32))
    zeros = np.floor(rng.uniform(0, 8, (d_out, ng))).astype(np.float32)
    if specials:
        flat_s, flat_z = scales.ravel(), zeros.ravel()
        sv = np.array([np.nan, np.inf, -np.inf, 7e4, 65520.0, 65519.0, 3e-8, 6e-8, 1e-5, -0.0, 2.9e-8, 1e30],
                      np.float32)
        sv = np.concatenate([sv, np.array([0x7F812345, 0xFFC00001], np.uint32).view(np.float32)])
        zv = np.array([np.nan, -1.0, -0.5, 0.99, 255.9, 256.0, 1e9, np.inf, -np.inf, 3.5], np.float32)
        ks, kz = min(sv.size, flat_s.size), min(zv.size, flat_z.size)
        flat_s[:ks] = sv[:ks]
        flat_z[:kz] = zv[:kz]
    perm = (rng.permutation(n) if act_order else np.arange(n)).astype(np.uint32)
    return cdclq.QLayer(d_out, n, g, perm, gbits, codes, scales, zeros)


def _oracle_pack(ql):
    return O.pack_layer(ql.codes, ql.scales, ql.zeros, ql.perm, ql.gbits, ql.group)


def _same_bits(a, b, label):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype, label
    if a.dtype == np.float32:
        an, bn = np.isnan(a), np.isnan(b)
        assert np.array_equal(an, bn), f"{label}: NaN positions differ"
        a, b = np.where(an, 0, a).view(np.uint32), np.where(bn, 0, b).view(np.uint32)
    bad = np.argwhere(a != b)
    assert bad.size == 0, f"{label}: {len(bad)} mismatches, first at {bad[0]}: gpu {a[tuple(bad[0])]} " \
                          f"oracle {b[tuple(bad[0])]}"


def _same_16(a, b, label):
    """F16 / BF16 bit patterns; NaN patterns compared as NaN only (see module docstring)."""
    a, b = a.astype(np.uint32), b.astype(np.uint32)
    exp_mask, man_mask = (0x7C00, 0x03FF) if label.endswith("F16") and not label.endswith("BF16") else (0x7F80, 0x7F)
    an = ((a & exp_mask) == exp_mask) & ((a & man_mask) != 0)
    bn = ((b & exp_mask) == exp_mask) & ((b & man_mask) != 0)
    assert np.array_equal(an, bn), f"{label}: NaN positions differ"
    bad = np.argwhere((a != b) & ~an)
    assert bad.size == 0, f"{label}: {len(bad)} mismatches, first at {bad[0]}"


CASES = [
    # n, g, d_out, gbits (None = random 1..8)
    (167, 32, 5, [8, 3, 3, 4, 2, 3]),  # the reference's round-trip layout
    (1, 1, 3, None),
    (7, 3, 4, None),
    (64, 64, 2, [4]),
    (100, 7, 9, None),
    (257, 16, 33, None),
    (515, 128, 17, [2, 8, 5, 1, 7]),
    (1000, 1000, 3, [3]),
    (4096, 128, 64, [4] * 32),
    (4096, 128, 48, [8, 8] + [3] * 30),
    (2050, 32, 31, None),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_pack_layer_matches_oracle(ctx, case):
    n, g, d_out, gb = CASES[case]
    print(f"[container] pack n={n} g={g} d_out={d_out}", flush=True)
    for wild, specials in ((False, False), (True, True)):
        ql = _layer(n, g, d_out, 1000 + case, wild=wild, specials=specials, gb=gb)
        got = cdclq.pack_layer(ctx, ql)
        ref = _oracle_pack(ql)
        for a, b, nm in zip(got, ref, ("qweight", "scales", "qzeros", "perm")):
            _same_bits(a, b, f"case {case} wild={wild} {nm}")


@pytest.mark.parametrize("case", range(len(CASES)))
def test_dequantize_packed_matches_oracle(ctx, case):
    n, g, d_out, gb = CASES[case]
    print(f"[container] dequant n={n} g={g} d_out={d_out}", flush=True)
    ql = _layer(n, g, d_out, 2000 + case, gb=gb)
    qw, s16, qz, p32 = _oracle_pack(ql)
    for dt in ("F32", "F16", "BF16"):
        got = cdclq.dequantize_packed(ctx, qw, s16, qz, p32, ql.gbits, g, dt)
        ref = O.dequantize_packed(qw, s16, qz, p32, ql.gbits, g, dt)
        _same_bits(got, ref, f"case {case} {dt}")


@pytest.mark.parametrize("case", [0, 4, 6, 10])
def test_dequantize_special_scales_and_zeros(ctx, case):
    """Scales that overflow f16, subnormal f16 scales, infinities, zero points outside 0..255."""
    n, g, d_out, gb = CASES[case]
    ql = _layer(n, g, d_out, 3000 + case, specials=True, gb=gb)
    qw, s16, qz, p32 = _oracle_pack(ql)
    for dt in ("F32", "F16", "BF16"):
        got = cdclq.dequantize_packed(ctx, qw, s16, qz, p32, ql.gbits, g, dt)
        ref = O.dequantize_packed(qw, s16, qz, p32, ql.gbits, g, dt)
        if dt == "F32":
            _same_bits(got, ref, f"special {case} F32")
        else:
            _same_16(got, ref, f"special {case} {dt}")


@pytest.mark.parametrize("case", [0, 2, 5, 8])
def test_dequantize_layer_matches_oracle(ctx, case):
    n, g, d_out, gb = CASES[case]
    ql = _layer(n, g, d_out, 4000 + case, gb=gb)
    ref32 = O.QLayer(d_out, n, g, ql.perm, ql.gbits, ql.codes, ql.scales, ql.zeros, {}).dequantize()
    for dt in ("F32", "F16", "BF16"):
        got = cdclq.dequantize_layer(ctx, ql, dt)
        _same_bits(got, O.narrow(ref32, dt), f"layer case {case} {dt}")


def _f32_classes(count, seed):
    """Random f32 bit patterns plus the cases that decide a rounding: every f16 / bf16 tie and its
    neighbours over the whole exponent range, f16 overflow, subnormals, zeros, infinities, NaNs."""
    rng = np.random.default_rng(seed)
    u = rng.integers(0, 1 << 32, count, dtype=np.uint64).astype(np.uint32)
    sp = []
    for e in range(0, 255):
        for m in (0, 1, 0x0FFF, 0x1000, 0x1001, 0x3000, 0x7FFF, 0x8000, 0x8001, 0x18000, 0x7FFFFF, 0x7FE000,
                  0x7FF000, 0x7FEFFF):
            sp.append((e << 23) | m)
    sp += [0x7F800000, 0x7F800001, 0x7FC00000, 0x7FFFFFFF, 0x7F812345]
    sp = np.array(sp, np.uint32)
    return np.concatenate([np.concatenate([sp, sp | 0x80000000]), u])


def test_narrowing_matches_half_for_every_value_class(ctx):
    """io::f32_to_bytes (src/io.rs:50-57) on the device: dequantize_layer with one column per group,
    code 1 and zero 0 passes each scale through unchanged (s * (1 - 0) = s), so the F16 / BF16
    outputs are exactly the narrowing of arbitrary f32 patterns."""
    n = 4096
    vals = _f32_classes(4096 * n - 2 * 255 * 14 - 10, 9)
    d_out = vals.size // n
    scales = vals[: d_out * n].view(np.float32).reshape(d_out, n)
    ql = cdclq.QLayer(d_out, n, 1, np.arange(n, dtype=np.uint32), np.full(n, 8, np.uint8),
                      np.ones((d_out, n), np.uint8), scales, np.zeros((d_out, n), np.float32))
    for dt in ("F32", "F16", "BF16"):
        got = cdclq.dequantize_layer(ctx, ql, dt)
        with np.errstate(invalid="ignore"):
            ref = O.narrow(scales * np.float32(1.0), dt)
        if dt == "F32":
            _same_bits(got, ref, "narrow F32")
        else:
            _same_16(got, ref, f"narrow {dt}")


def test_repeated_perm_entries_keep_the_scatter_result(ctx):
    ql = _layer(300, 128, 6, 77)
    ql.perm[5] = ql.perm[17]
    ql.perm[200] = ql.perm[17]
    qw, s16, qz, p32 = _oracle_pack(ql)
    got = cdclq.dequantize_packed(ctx, qw, s16, qz, p32, ql.gbits, 128, "F32")
    _same_bits(got, O.dequantize_packed(qw, s16, qz, p32, ql.gbits, 128, "F32"), "dup perm")


def test_device_entry_points_match_host(ctx):
    ql = _layer(4096, 128, 40, 9, gb=[4] * 32)
    d_out, n, g, ng = ql.d_out, ql.d_in, ql.group, ql.ngroups()
    rb = cdclq.row_bytes(n, g, ql.gbits)
    host = cdclq.pack_layer(ctx, ql)
    dc = cdclq.DeviceArray.from_host(ctx, ql.codes)
    ds = cdclq.DeviceArray.from_host(ctx, ql.scales)
    dz = cdclq.DeviceArray.from_host(ctx, ql.zeros)
    dp = cdclq.DeviceArray.from_host(ctx, ql.perm)
    dq = cdclq.DeviceArray(ctx, (d_out, rb), np.uint8)
    d16 = cdclq.DeviceArray(ctx, (d_out, ng), np.uint16)
    d8 = cdclq.DeviceArray(ctx, (d_out, ng), np.uint8)
    d32 = cdclq.DeviceArray(ctx, (n,), np.int32)
    gb = np.ascontiguousarray(ql.gbits, np.uint8)
    L = cdclq.lib()
    ctx.check(L.cdclq_pack_layer_device(ctx.ptr, d_out, n, g, gb.ctypes.data, ng, dc.ptr, ds.ptr, dz.ptr, dp.ptr,
                                        dq.ptr, d_out * rb, d16.ptr, d8.ptr, d32.ptr))
    for a, b, nm in zip((dq.download(), d16.download(), d8.download(), d32.download()), host,
                        ("qweight", "scales", "qzeros", "perm")):
        _same_bits(a, b, f"device {nm}")
    out = cdclq.DeviceArray(ctx, (d_out, n), np.uint16)
    ctx.check(L.cdclq_dequantize_packed_device(ctx.ptr, d_out, n, g, gb.ctypes.data, ng, dq.ptr, d_out * rb,
                                               d16.ptr, d8.ptr, d32.ptr, cdclq.DTYPE_BF16, out.ptr))
    _same_bits(out.download(), cdclq.dequantize_packed(ctx, *host, ql.gbits, g, "BF16"), "device dequant")
    out32 = cdclq.DeviceArray(ctx, (d_out, n), np.float32)
    ctx.check(L.cdclq_dequantize_layer_device(ctx.ptr, d_out, n, g, ng, dc.ptr, ds.ptr, dz.ptr, dp.ptr,
                                              cdclq.DTYPE_F32, out32.ptr))
    _same_bits(out32.download(), cdclq.dequantize_layer(ctx, ql, "F32"), "device layer dequant")
    for a in (dc, ds, dz, dp, dq, d16, d8, d32, out, out32):
        a.free()


def test_invalid_layouts_are_rejected(ctx):
    ql = _layer(100, 32, 3, 5, gb=[4, 4, 4, 4])
    qw, s16, qz, p32 = _oracle_pack(ql)
    bad = [
        (dict(gbits=np.array([4, 4, 4], np.uint8)), "ngroups"),
        (dict(gbits=np.array([4, 0, 4, 4], np.uint8)), "1..=8"),
        (dict(gbits=np.array([4, 9, 4, 4], np.uint8)), "1..=8"),
        (dict(group=0), "group size"),
    ]
    for kw, frag in bad:
        args = dict(gbits=ql.gbits, group=32)
        args.update(kw)
        with pytest.raises(cdclq.CdclqError) as e:
            cdclq.dequantize_packed(ctx, qw, s16, qz, p32, args["gbits"], args["group"], "F32")
        assert e.value.code == cdclq.INVALID_ARG and frag in str(e.value), str(e.value)
    p_bad = p32.copy()
    p_bad[3] = 100
    with pytest.raises(cdclq.CdclqError) as e:
        cdclq.dequantize_packed(ctx, qw, s16, qz, p_bad, ql.gbits, 32, "F32")
    assert "perm" in str(e.value)
    p_bad[3] = -1
    with pytest.raises(cdclq.CdclqError):
        cdclq.dequantize_packed(ctx, qw, s16, qz, p_bad, ql.gbits, 32, "F32")
    with pytest.raises(cdclq.CdclqError) as e:
        cdclq.dequantize_packed(ctx, qw[:, :-1], s16, qz, p32, ql.gbits, 32, "F32")
    assert "qweight" in str(e.value)
    with pytest.raises(cdclq.CdclqError) as e:
        cdclq.dequantize_packed(ctx, qw, s16, qz, p32, ql.gbits, 32, 7)
    assert "dtype" in str(e.value)
    # the context stays usable after the errors
    got = cdclq.dequantize_packed(ctx, qw, s16, qz, p32, ql.gbits, 32, "F32")
    _same_bits(got, O.dequantize_packed(qw, s16, qz, p32, ql.gbits, 32, "F32"), "after errors")


def test_engine_output_roundtrips_through_the_container(ctx):
    """src/io.rs via tests/toy_models.rs:290-320: every quantized layer unpacks through the reader
    path to exactly what QLayer::dequantize wrote, and both equal the oracle's."""
    w, x, h, _ = synth_layer(11, 64, 384, 1200)
    cfg = cdclq.Config(bits=3, group=64, block=64, act_order=True, skeleton_pct=25.0, skeleton_bits=5, passes=2,
                       row_chunk=16)
    ql, st = cdclq.quantize_layer(w, 64, 384, h, None, "rt", cfg, cdclq.PrepCache(ctx=ctx))
    assert st.skeleton_groups > 0 and len(set(ql.gbits.tolist())) == 2
    tensors = cdclq.packed_tensors("model.layers.0.mlp.up_proj", ql, ctx)
    assert tensors["model.layers.0.mlp.up_proj.qweight"][1].shape == (64, cdclq.row_bytes(384, 64, ql.gbits))
    for dt in ("F32", "F16", "BF16"):
        via_reader = cdclq.read_packed_dequantized(tensors, "model.layers.0.mlp.up_proj", ctx, dt)
        direct = cdclq.dequantize_layer(ctx, ql, dt)
        _same_bits(via_reader, direct, f"reader vs dequant {dt}")
    ref = O.dequantize_packed(*_oracle_pack(ql), ql.gbits, ql.group, "F32")
    _same_bits(cdclq.dequantize_layer(ctx, ql, "F32"), ref, "engine layer vs oracle")


def test_llama3_8b_down_proj_shape(ctx):
    """Full-size layer (14336 x 4096 codes would be up_proj's; down_proj is 4096 x 14336): 4-bit,
    group 128, act-order, against the oracle byte for byte."""
    d_out, n, g = 4096, 14336, 128
    ql = _layer(n, g, d_out, 8, gb=[4] * (n // g))
    print(f"[container] full size {d_out}x{n}", flush=True)
    got = cdclq.pack_layer(ctx, ql)
    ref = _oracle_pack(ql)
    for a, b, nm in zip(got, ref, ("qweight", "scales", "qzeros", "perm")):
        _same_bits(a, b, f"full {nm}")
    out = cdclq.dequantize_packed(ctx, *got, ql.gbits, g, "BF16")
    _same_bits(out, O.dequantize_packed(*ref, ql.gbits, g, "BF16"), "full BF16")


def test_widest_rows_use_more_than_64k_of_lds(ctx):
    """Rows of 65536 8-bit codes (packed) and 131072 u8 codes (unpacked) need > 64 KiB of LDS."""
    for n, g, d_out in ((65536, 128, 3), (131072, 4096, 2)):
        print(f"[container] wide rows n={n}", flush=True)
        ql = _layer(n, g, d_out, n, gb=[8] * (n // g))
        qw, s16, qz, p32 = _oracle_pack(ql)
        got = cdclq.dequantize_packed(ctx, qw, s16, qz, p32, ql.gbits, g, "F32")
        _same_bits(got, O.dequantize_packed(qw, s16, qz, p32, ql.gbits, g, "F32"), f"wide packed {n}")
        ref32 = O.QLayer(d_out, n, g, ql.perm, ql.gbits, ql.codes, ql.scales, ql.zeros, {}).dequantize()
        _same_bits(cdclq.dequantize_layer(ctx, ql, "F32"), ref32, f"wide layer {n}")

"""Pins of the oracle's packed-container restatement (cdclq-v1: src/quant.rs:98-236,
src/io.rs:50-57, :244-293) and of the `half` 2.4.1 conversions it relies on.

Each check is an independent formulation, not the oracle's own loop retyped:
  * the reference's own round-trip test (src/quant.rs:259-275), same Rng(9) codes;
  * a row as one Python integer: OR over j of code_j << off_j, little-endian bytes (this also
    fixes the reference's unmasked OR of out-of-range codes);
  * numpy.packbits(bitorder="little") of each code's low bits;
  * numpy float16 (IEEE RNE) and torch bfloat16 conversions for the narrowing;
  * numpy float32 arithmetic and fancy-index scatter for QLayer::dequantize.
Planted mistakes (oracle mutations 9 and 10) must fail them.
"""
import numpy as np
import pytest
import torch

import oracle as O


def _offsets(n, g, gbits):
    w = np.asarray(gbits, np.int64)[np.arange(n) // g]
    off = np.concatenate([[0], np.cumsum(w)])
    return off[:-1], w, int(off[-1])


def _bigint_row(codes, n, g, gbits):
    off, _, total = _offsets(n, g, gbits)
    v = 0
    for j in range(n):
        v |= int(codes[j]) << int(off[j])
    rb = (total + 7) // 8
    return np.frombuffer(v.to_bytes(rb + 2, "little")[:rb], np.uint8)


def _packbits_row(codes, n, g, gbits):
    _, w, total = _offsets(n, g, gbits)
    bits = np.unpackbits(np.asarray(codes, np.uint8)[:, None], axis=1, bitorder="little")
    stream = np.concatenate([bits[j, : w[j]] for j in range(n)]) if n else np.zeros(0, np.uint8)
    return np.packbits(stream, bitorder="little")


def _layouts():
    rng = np.random.default_rng(5)
    out = [(167, 32, np.array([8, 3, 3, 4, 2, 3], np.uint8))]  # the reference's own case
    for n, g in [(1, 1), (7, 3), (64, 64), (100, 7), (300, 128), (257, 16), (1000, 1000), (515, 128)]:
        ng = (n + g - 1) // g
        out.append((n, g, rng.integers(1, 9, ng).astype(np.uint8)))
    out.append((4096, 128, np.full(32, 4, np.uint8)))
    out.append((4096, 128, np.array([8, 8] + [3] * 30, np.uint8)))
    return out


def test_reference_roundtrip_mixed_bits():
    """src/quant.rs:259-275: mixed widths in one row, ragged last group, Rng(9) codes."""
    r = O.Rng(9)
    g, n = 32, 32 * 5 + 7
    gbits = np.array([8, 3, 3, 4, 2, 3], np.uint8)
    codes = np.array([r.next_u64() % (1 << int(gbits[j // g])) for j in range(n)], np.uint8)
    rb = O.row_bytes(n, g, gbits)
    assert rb == (32 * (8 + 3 + 3 + 4 + 2) + 7 * 3 + 7) // 8
    buf = O.pack_row(codes, g, gbits)
    assert buf.size == rb
    np.testing.assert_array_equal(O.unpack_row(buf, n, g, gbits), codes)


@pytest.mark.parametrize("case", range(len(_layouts())))
def test_pack_row_is_the_lsb_first_bitstream(case):
    n, g, gbits = _layouts()[case]
    rng = np.random.default_rng(100 + case)
    _, w, _ = _offsets(n, g, gbits)
    codes = (rng.integers(0, 1 << 8, n) & ((1 << w) - 1)).astype(np.uint8)
    buf = O.pack_row(codes, g, gbits)
    np.testing.assert_array_equal(buf, _bigint_row(codes, n, g, gbits))
    np.testing.assert_array_equal(buf, _packbits_row(codes, n, g, gbits))
    np.testing.assert_array_equal(O.unpack_row(buf, n, g, gbits), codes)
    # out-of-range codes: the reference ORs the whole u8 into its accumulator
    wild = rng.integers(0, 256, n).astype(np.uint8)
    np.testing.assert_array_equal(O.pack_row(wild, g, gbits), _bigint_row(wild, n, g, gbits))


def test_unpack_extracts_each_code_from_its_offset():
    n, g, gbits = 515, 128, np.array([2, 8, 5, 1, 7], np.uint8)
    off, w, total = _offsets(n, g, gbits)
    data = np.random.default_rng(3).integers(0, 256, (total + 7) // 8).astype(np.uint8)
    v = int.from_bytes(data.tobytes(), "little")
    expect = np.array([(v >> int(off[j])) & ((1 << int(w[j])) - 1) for j in range(n)], np.uint8)
    np.testing.assert_array_equal(O.unpack_row(data, n, g, gbits), expect)


@pytest.mark.parametrize("mid", [9, 10])
def test_planted_packing_mistakes_are_caught(mid):
    n, g, gbits = 167, 32, np.array([8, 3, 3, 4, 2, 3], np.uint8)
    rng = np.random.default_rng(11)
    wild = rng.integers(0, 256, n).astype(np.uint8)
    _, w, _ = _offsets(n, g, gbits)
    tame = (wild & ((1 << w) - 1)).astype(np.uint8)
    with O.mutation(mid):
        a = O.pack_row(wild, g, gbits)
        b = O.pack_row(tame, g, gbits)
    assert not (np.array_equal(a, _bigint_row(wild, n, g, gbits)) and np.array_equal(b, _packbits_row(tame, n, g, gbits)))


def _f32_patterns(count, seed):
    rng = np.random.default_rng(seed)
    u = rng.integers(0, 1 << 32, count, dtype=np.uint64).astype(np.uint32)
    special = []
    for e in range(90, 150):  # around the f16 range, incl. ties at every binary16 exponent
        for m in (0, 0x1000, 0x2000 | 0x1000, 0x0fff, 0x1001, 0x7fffff, 0x8000, 0x18000, 0x7fff):
            special.append((e << 23) | m)
    special += [0, 0x80000000, 0x7F800000, 0xFF800000, 0x477FE000, 0x477FF000, 0x477FEFFF, 0x33000000,
                0x33000001, 0x337FFFFF, 0x7F7FFFFF, 0x00000001, 0x3F808000, 0x3F818000, 0x3F80FFFF]
    s = np.array(special, np.uint32)
    return np.concatenate([u, s, s | 0x80000000])


def test_f16_narrowing_matches_ieee_rne():
    u = _f32_patterns(1 << 22, 1)
    x = u.view(np.float32)
    got = O.narrow(x, "F16")
    fin = ~np.isnan(x)
    with np.errstate(over="ignore"):
        ref = x[fin].astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got[fin], ref)
    # NaN: sign and the upper 10 payload bits kept, quiet bit set (half 2.4.1 / F16C)
    nan = u[~fin]
    g = got[~fin].astype(np.uint32)
    assert ((g & 0x7C00) == 0x7C00).all() and ((g & 0x0200) != 0).all()
    np.testing.assert_array_equal(g & 0x8000, (nan >> 16) & 0x8000)
    np.testing.assert_array_equal(g & 0x1FF, (nan >> 13) & 0x1FF)


def test_f16_widening_is_exact_for_every_pattern():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = np.array([O.lib().orc_f16_bits_to_f32(int(v)) for v in h], np.float32)
    ref = h.view(np.float16).astype(np.float32)
    fin = ~np.isnan(ref)
    np.testing.assert_array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    gn = got[~fin].view(np.uint32)
    assert ((gn & 0x00400000) != 0).all() and np.isnan(got[~fin]).all()


def test_bf16_narrowing_matches_torch_rne():
    u = _f32_patterns(1 << 22, 2)
    x = u.view(np.float32)
    got = O.narrow(x, "BF16")
    fin = ~np.isnan(x)
    ref = torch.from_numpy(x[fin].copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got[fin], ref)
    nan = u[~fin]
    g = got[~fin].astype(np.uint32)
    np.testing.assert_array_equal(g, ((nan >> 16) | 0x40) & 0xFFFF)


def test_zero_points_are_saturating_u8_casts():
    z = np.array([0.0, -0.0, 0.7, 1.0, 3.999, 7.0, 254.9, 255.0, 255.5, 1e9, -1.5, -1e9, np.inf, -np.inf, np.nan],
                 np.float32)
    expect = [0, 0, 0, 1, 3, 7, 254, 255, 255, 255, 0, 0, 255, 0, 0]
    qw, s16, qz, p32 = O.pack_layer(np.zeros((1, z.size), np.uint8), np.ones((1, z.size), np.float32), z[None, :],
                                    np.arange(z.size, dtype=np.uint32), np.full(z.size, 2, np.uint8), 1)
    assert qz.ravel().tolist() == expect
    np.testing.assert_array_equal(p32, np.arange(z.size))


def _numpy_dequant(qw, s16, qz, p32, gbits, g, n):
    off, w, _ = _offsets(n, g, gbits)
    d_out = qw.shape[0]
    codes = np.zeros((d_out, n), np.uint8)
    for r in range(d_out):
        v = int.from_bytes(qw[r].tobytes(), "little")
        codes[r] = [(v >> int(off[j])) & ((1 << int(w[j])) - 1) for j in range(n)]
    gi = np.arange(n) // g
    s = s16.view(np.float16).astype(np.float32)[:, gi]
    z = qz.astype(np.float32)[:, gi]
    vals = s * (codes.astype(np.float32) - z)
    out = np.zeros((d_out, n), np.float32)
    out[:, p32.astype(np.int64)] = vals
    return out


@pytest.mark.parametrize("n,g,dup", [(300, 128, False), (167, 32, False), (515, 7, True), (64, 64, False)])
def test_dequantize_packed_matches_numpy(n, g, dup):
    rng = np.random.default_rng(n + g)
    d_out = 9
    ng = (n + g - 1) // g
    gbits = rng.integers(2, 9, ng).astype(np.uint8)
    _, w, _ = _offsets(n, g, gbits)
    codes = (rng.integers(0, 256, (d_out, n)) & ((1 << w) - 1)).astype(np.uint8)
    scales = O.round_f16(rng.uniform(1e-3, 0.5, (d_out, ng)).astype(np.float32))
    zeros = np.floor(rng.uniform(0, 7, (d_out, ng))).astype(np.float32)
    perm = rng.permutation(n).astype(np.uint32)
    if dup:
        perm[5] = perm[17]  # the reference's scatter: the later j wins, one column stays 0
    qw, s16, qz, p32 = O.pack_layer(codes, scales, zeros, perm, gbits, g)
    ref = _numpy_dequant(qw, s16, qz, p32, gbits, g, n)
    np.testing.assert_array_equal(O.dequantize_packed(qw, s16, qz, p32, gbits, g, "F32").view(np.uint32),
                                  ref.view(np.uint32))
    np.testing.assert_array_equal(O.dequantize_packed(qw, s16, qz, p32, gbits, g, "F16"),
                                  ref.astype(np.float16).view(np.uint16))
    np.testing.assert_array_equal(O.dequantize_packed(qw, s16, qz, p32, gbits, g, "BF16"),
                                  torch.from_numpy(ref).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
    # the unpacked path (QLayer::dequantize) agrees with the packed one when scales are f16-exact
    ql = O.QLayer(d_out, n, g, perm, gbits, codes, scales, zeros, {})
    np.testing.assert_array_equal(ql.dequantize().view(np.uint32), ref.view(np.uint32))

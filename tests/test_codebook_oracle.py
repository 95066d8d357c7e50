"""The codebook weight format's oracle pinned against closed forms.

The reference's own tests for this path (crates/kernels/tests/walsh.rs,
quantised_matrix.rs) need the model archives for everything but the transform;
the archives are not in the reference tree, so the product is pinned here by
what the mathematics fixes:
  - the transform against the dense normalised Hadamard matrix (walsh.rs:1-31)
    and by applying it twice (walsh.rs:33-40);
  - index unpacking (LSB first) and the integer table on hand-made bytes;
  - the exact int32 group sums against an int64 brute force over unpacked
    indices;
  - the float product against the dense dequantised matrix times the
    unrotated input (the identity H = H^T behind quantised_matrix.rs:36-55;
    the reference allows 2% relative RMS there, the input quantisation
    costs about 1%), which fails for a wrong rotation, packing, table, norm
    or epilogue;
  - dequantise_row against (level x norm) times the dense Hadamard matrix.
"""
from fractions import Fraction

import numpy as np
import pytest

import oracle
import rustyneedle_amd as rn


def hadamard(n: int) -> np.ndarray:
    i = np.arange(n)
    signs = np.array([[1 - 2 * (bin(r & c).count("1") % 2) for c in i] for r in i], dtype=np.float64)
    return signs / np.sqrt(n)


@pytest.mark.parametrize("size", [4, 8, 32, 64, 128, 256])
def test_transform_matches_the_dense_hadamard_matrix(size):
    x = np.array([(((i * 7919 + size) % 2003) - 1000.0) / 400.0 for i in range(size)], np.float32)
    got = oracle.walsh_transform(x).astype(np.float64)
    want = hadamard(size) @ x.astype(np.float64)
    assert np.max(np.abs(got - want) / (1.0 + np.abs(want))) < 1e-5


def test_transform_twice_returns_the_input():
    x = np.sin(np.arange(128, dtype=np.float32) * np.float32(0.37)).astype(np.float32)
    assert np.max(np.abs(oracle.walsh_transform(oracle.walsh_transform(x)) - x)) < 1e-5


def test_transform_of_a_unit_vector_is_a_signed_constant():
    for k in (0, 5, 127):
        e = np.zeros(128, np.float32)
        e[k] = 1.0
        got = oracle.walsh_transform(e)
        scale = np.float32(1.0) / np.sqrt(np.float32(128.0))
        assert np.array_equal(np.abs(got), np.full(128, scale, np.float32))
        assert np.array_equal(np.sign(got), np.sign(hadamard(128)[:, k]))


def test_prepare_pads_with_zeros_and_rotates_each_group():
    x = np.arange(1, 101, dtype=np.float32)
    r = oracle.codebook_prepare(x, 128, 64)
    full = np.zeros(128, np.float32)
    full[:100] = x
    assert np.array_equal(r[:64], oracle.walsh_transform(full[:64]))
    assert np.array_equal(r[64:], oracle.walsh_transform(full[64:]))


def test_integer_levels_round_half_away_from_zero():
    levels = np.zeros(16, np.float32)
    levels[:4] = [-127.0, -2.5, 2.5, 0.5]  # scale 127/127 = 1: 2.5 -> 3 (ties-even would give 2)
    table, scale = oracle.integer_levels(levels, 4)
    assert scale == np.float32(1.0)
    assert table[:4].tolist() == [-127, -3, 3, 1]
    assert table[4:].tolist() == [0] * 12
    table, scale = oracle.integer_levels(np.zeros(16, np.float32), 4)
    assert scale == np.float32(1.0) and table.tolist() == [0] * 16


def test_codebook_levels_by_width():
    cb = rn.synthetic_codebook(128)
    lv, n = oracle.codebook_levels(cb, 2, 128)
    assert n == 4 and np.array_equal(lv[:4], cb[:4]) and not lv[4:].any()
    lv, n = oracle.codebook_levels(cb, 4, 128)
    assert n == 16 and np.array_equal(lv, cb[12:28])
    lv, n = oracle.codebook_levels(cb, 5, 128)
    level = np.float32(1.2240064) / np.sqrt(np.float32(128))
    assert n == 4 and lv[:4].tolist() == [0.0, level, 0.0, -level]
    table, _ = oracle.integer_levels(lv, n)
    assert table[:4].tolist() == [0, 127, 0, -127]


def _unpack(packed: np.ndarray, rows: int, padded: int, ib: int) -> np.ndarray:
    bits = np.unpackbits(packed.reshape(rows, -1), axis=1, bitorder="little").reshape(rows, padded, ib)
    return (bits * (1 << np.arange(ib))).sum(axis=2)


def test_indices_are_least_significant_bits_first():
    cb = rn.synthetic_codebook(64)
    blob = np.zeros(64 // 4 + 2, np.uint8)  # one 64-wide row of 2-bit indices and one norm
    blob[0] = 0b11100100  # elements 0..3 -> indices 0, 1, 2, 3
    blob[16:18] = np.array([1.0], np.float16).view(np.uint8)
    m = oracle.OracleCodebookMatrix(blob, 1, 64, 64, 2, cb)
    row = m.dequantise_row(0)
    c = np.zeros(64, np.float32)
    c[:4] = cb[:4]
    c[4:] = cb[0]
    assert np.allclose(row, hadamard(64) @ c, atol=1e-6)
    assert _unpack(blob[:16], 1, 64, 2)[0, :4].tolist() == [0, 1, 2, 3]
    four = np.array([0xA3], np.uint8)
    assert _unpack(np.concatenate([four, np.zeros(31, np.uint8)]), 1, 64, 4)[0, :2].tolist() == [3, 10]


CASES = [(2, 64, 96, 200), (2, 128, 64, 512), (4, 128, 48, 384), (4, 64, 40, 130), (5, 128, 32, 256),
         (2, 256, 24, 700), (4, 256, 16, 512)]


@pytest.mark.parametrize("bits,group,rows,columns", CASES)
def test_integer_sums_match_a_brute_force(bits, group, rows, columns):
    cb = rn.synthetic_codebook(group)
    blob = rn.synthetic_codebook_blob(rows, columns, group, bits, seed=3)
    m = oracle.OracleCodebookMatrix(blob, rows, columns, group, bits, cb)
    x = rn.synth_normal(7, "cb.x", 1.0, (2, columns))
    rotated = np.stack([m.prepare(v) for v in x])
    y, acc = m.multiply_rotated(rotated, with_acc=True)
    ib = 2 if bits == 5 else bits
    idx = _unpack(m.packed, rows, m.padded, ib)
    w = m.table[idx].astype(np.int64)
    for t in range(2):
        codes, _ = oracle.group_codes(rotated[t], group)
        prod = (w * codes.astype(np.int64)[None, :]).reshape(rows, -1, group).sum(axis=2)
        assert np.array_equal(acc[t], prod)


@pytest.mark.parametrize("bits,group,rows,columns", CASES)
def test_product_matches_the_dense_dequantised_matrix(bits, group, rows, columns):
    cb = rn.synthetic_codebook(group)
    blob = rn.synthetic_codebook_blob(rows, columns, group, bits, seed=4)
    m = oracle.OracleCodebookMatrix(blob, rows, columns, group, bits, cb)
    x = rn.synth_normal(9, "cb.x", 1.0, (columns,))
    y = m.multiply(x)[0].astype(np.float64)
    ib = 2 if bits == 5 else bits
    idx = _unpack(m.packed, rows, m.padded, ib)
    norms = m.norms.view(np.float16).astype(np.float64).reshape(rows, -1)
    lv = m.levels.astype(np.float64)[idx] * np.repeat(norms, group, axis=1)
    H = hadamard(group)
    dense = np.concatenate([lv[:, g * group:(g + 1) * group] @ H for g in range(m.padded // group)], axis=1)
    want = dense[:, :columns] @ x.astype(np.float64)
    rel = np.sqrt(np.sum((y - want) ** 2) / np.sum(want ** 2))
    assert rel < 0.02, rel
    assert np.allclose(np.stack([m.dequantise_row(r) for r in range(rows)]), dense[:, :columns], atol=1e-5)


def test_zero_input_gives_zero_rows():
    cb = rn.synthetic_codebook(128)
    m = oracle.OracleCodebookMatrix(rn.synthetic_codebook_blob(8, 256, 128, 2), 8, 256, 128, 2, cb)
    y, acc = m.multiply(np.zeros(256, np.float32), with_acc=True)
    assert not y.any() and not acc.any()
    codes, scales = oracle.group_codes(np.zeros(256, np.float32), 128)
    assert np.all(scales == 1.0) and not codes.any()


def _round_f32(fr):
    """Correctly rounded (nearest, ties to even) float32 of an exact rational."""
    x = np.float32(float(fr))
    best = x
    for cand in (np.nextafter(x, np.float32(-np.inf)), np.nextafter(x, np.float32(np.inf))):
        d_best, d_cand = abs(Fraction(float(best)) - fr), abs(Fraction(float(cand)) - fr)
        if d_cand < d_best or (d_cand == d_best and (int(cand.view(np.uint32)) & 1) == 0):
            best = cand
    return np.float32(best)


def _epilogue_inputs(bits, rows=96, columns=512, group=128):
    cb = rn.synthetic_codebook(group)
    m = oracle.OracleCodebookMatrix(rn.synthetic_codebook_blob(rows, columns, group, bits, seed=21), rows, columns,
                                    group, bits, cb)
    rotated = m.prepare(rn.synth_normal(22, "cb.x", 1.0, (columns,)))
    y, acc = m.multiply_rotated(rotated, with_acc=True)
    _, xs = oracle.group_codes(rotated, group)
    norms = m.norms.view(np.float16).astype(np.float32).reshape(rows, -1)
    return m, y[0], acc[0], xs, norms


def test_two_bit_epilogue_is_the_panel_fma():
    """panel.rs:184-188: total = fma(acc, (norm * lscale) * xs, total), one
    rounding per group; rows where two roundings differ make the check bite."""
    m, y, acc, xs, norms = _epilogue_inputs(2)
    differs = 0
    for r in range(m.rows):
        fused = unfused = np.float32(0)
        for g in range(m.padded // m.group):
            s = np.float32(np.float32(norms[r, g] * m.lscale) * xs[g])
            fused = _round_f32(Fraction(int(acc[r, g])) * Fraction(float(s)) + Fraction(float(fused)))
            unfused = np.float32(unfused + np.float32(np.float32(acc[r, g]) * s))
        assert y[r] == fused, r
        differs += int(fused != unfused)
    assert differs > 0


@pytest.mark.parametrize("bits", [4, 5])
def test_plane_epilogue_sequential_order(bits):
    """neon.rs:158,180: total += acc as f32 * norm * lscale * xs, left to right in
    float32; the panel fma differs on some rows, so the check bites."""
    m, y, acc, xs, norms = _epilogue_inputs(bits)
    differs = 0
    for r in range(m.rows):
        total = fused = np.float32(0)
        for g in range(m.padded // m.group):
            a = np.float32(acc[r, g])
            total = np.float32(total + np.float32(np.float32(np.float32(a * norms[r, g]) * m.lscale) * xs[g]))
            s = np.float32(np.float32(norms[r, g] * m.lscale) * xs[g])
            fused = _round_f32(Fraction(int(acc[r, g])) * Fraction(float(s)) + Fraction(float(fused)))
        assert y[r] == total, r
        differs += int(fused != total)
    assert differs > 0

"""The float path of the codebook format: fill_rows_float / LookupTable::dot_group
(crates/kernels/src/matrix.rs:427-440, 610-620) and multiply_batch's float tile
(matrix.rs:356-378, expand_row_scaled :390-399, dot :488-497) — the products
the reference computes on x86-64 for every width and everywhere for 1- and
3-bit matrices.

The oracle is pinned by:
- the mathematics: both orders agree with the float64 product of the
  dequantised levels (level * fp16 norm) and the rotated input to float32
  rounding, for widths 1-5 and groups 64-256;
- the index decoding, exactly: an input with one non-zero element returns
  level * norm of that element bit for bit, read from the packed bits by an
  independent decoder (including 3-bit indices that straddle two bytes);
- the summation orders: inputs built so that the per-byte lanes, the
  positional 3-bit sum and the eight-lane dot give different bits than a plain
  left-to-right sum, compared with a NumPy float32 reduction written per
  the reference's loops (the orders are the reference's, read from its source).
GPU tests (marked gpu) compare the device kernels with the oracle bit for bit.
"""
import numpy as np
import pytest

import oracle
import rustyneedle_amd as rn

WIDTHS = (1, 2, 3, 4, 5)


def _matrix(rows, columns, group, bits, seed):
    cb = rn.synthetic_codebook(group)
    blob = rn.synthetic_codebook_blob(rows, columns, group, bits, seed=seed, name=f"float.{bits}.{group}")
    return blob, cb, oracle.OracleCodebookMatrix(blob, rows, columns, group, bits, cb)


def _decode(om, row):
    """Independent decode: the row's index of every element (LSB first across bytes)."""
    ib = 2 if om.bits == 5 else om.bits
    row_bytes = om.padded * ib // 8
    raw = om.packed[row * row_bytes:(row + 1) * row_bytes]
    bits = np.unpackbits(raw, bitorder="little")
    idx = bits[:om.padded * ib].reshape(om.padded, ib)
    return (idx * (1 << np.arange(ib))).sum(axis=1)


def _dense(om):
    levels = om.levels.astype(np.float64)
    norms = om.norms.view(np.float16).astype(np.float64).reshape(om.rows, om.padded // om.group)
    return np.stack([levels[_decode(om, r)] * np.repeat(norms[r], om.group) for r in range(om.rows)])


@pytest.mark.parametrize("bits", WIDTHS)
@pytest.mark.parametrize("group", (64, 128, 256))
def test_float_path_against_float64(bits, group):
    rows, columns = 24, 3 * group - 17
    _, _, om = _matrix(rows, columns, group, bits, seed=bits * 7 + group)
    rng = np.random.default_rng(bits + group)
    rotated = rng.standard_normal((3, om.padded)).astype(np.float32)
    ref = rotated.astype(np.float64) @ _dense(om).T
    for batch in (False, True):
        y = om.multiply_float(rotated, batch=batch)
        assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref)), (bits, group, batch)


@pytest.mark.parametrize("bits", WIDTHS)
def test_single_element_decodes_exactly(bits):
    group = 64
    _, _, om = _matrix(5, 192, group, bits, seed=40 + bits)
    levels = om.levels
    norms = om.norms.view(np.float16).astype(np.float32).reshape(om.rows, om.padded // group)
    # element positions including 3-bit indices that straddle bytes (e = 2, 5, 10, 13 ...)
    for e in (0, 1, 2, 5, 7, 10, 13, 63, 64, 130, 191):
        x = np.zeros((1, om.padded), np.float32)
        x[0, e] = 1.0
        want = np.array([levels[_decode(om, r)[e]] * norms[r, e // group] for r in range(om.rows)], np.float32)
        for batch in (False, True):
            got = om.multiply_float(x, batch=batch)[0]
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (bits, e, batch)


def _reference_order_vector(om, rotated):
    """fill_rows_float over the reference's loops, in NumPy float32."""
    ib = 2 if om.bits == 5 else om.bits
    levels = om.levels.astype(np.float32)
    norms = om.norms.view(np.float16).astype(np.float32).reshape(om.rows, om.padded // om.group)
    out = np.empty((rotated.shape[0], om.rows), np.float32)
    for r in range(om.rows):
        lv = levels[_decode(om, r)]
        for t in range(rotated.shape[0]):
            total = np.float32(0.0)
            for g in range(om.padded // om.group):
                seg = (lv[g * om.group:(g + 1) * om.group] * rotated[t, g * om.group:(g + 1) * om.group]).astype(np.float32)
                if ib == 3:
                    partial = np.float32(-0.0)
                    for v in seg:
                        partial = np.float32(partial + v)
                else:
                    n = 8 // ib
                    lanes = np.zeros(n, np.float32)
                    for b in range(om.group // n):
                        lanes = (lanes + seg[b * n:(b + 1) * n]).astype(np.float32)
                    partial = np.float32(-0.0)
                    for v in lanes:
                        partial = np.float32(partial + v)
                total = np.float32(total + np.float32(partial * norms[r, g]))
            out[t, r] = total
    return out


def _reference_order_batch(om, rotated):
    """multiply_batch's float tile over the reference's loops, in NumPy float32."""
    levels = om.levels.astype(np.float32)
    norms = om.norms.view(np.float16).astype(np.float32).reshape(om.rows, om.padded // om.group)
    out = np.empty((rotated.shape[0], om.rows), np.float32)
    for r in range(om.rows):
        w = (levels[_decode(om, r)] * np.repeat(norms[r], om.group)).astype(np.float32)
        for t in range(rotated.shape[0]):
            prod = (w * rotated[t]).astype(np.float32).reshape(-1, 8)
            lanes = np.zeros(8, np.float32)
            for chunk in prod:
                lanes = (lanes + chunk).astype(np.float32)
            s = np.float32(-0.0)
            for v in lanes:
                s = np.float32(s + v)
            out[t, r] = s
    return out


@pytest.mark.parametrize("bits", WIDTHS)
def test_summation_orders(bits):
    group = 64
    _, _, om = _matrix(6, 128, group, bits, seed=90 + bits)
    rng = np.random.default_rng(bits)
    # magnitudes spread over many binades, so the order of the adds shows in the bits
    rotated = (rng.standard_normal((2, om.padded)) * 2.0 ** rng.integers(-12, 12, (2, om.padded))).astype(np.float32)
    v, b = om.multiply_float(rotated), om.multiply_float(rotated, batch=True)
    assert np.array_equal(v.view(np.uint32), _reference_order_vector(om, rotated).view(np.uint32))
    assert np.array_equal(b.view(np.uint32), _reference_order_batch(om, rotated).view(np.uint32))
    # and the orders matter for these inputs: a plain left-to-right row sum differs
    levels = om.levels.astype(np.float32)
    norms = om.norms.view(np.float16).astype(np.float32).reshape(om.rows, om.padded // om.group)
    plain = np.empty_like(v)
    for r in range(om.rows):
        w = (levels[_decode(om, r)] * np.repeat(norms[r], group)).astype(np.float32)
        for t in range(2):
            s = np.float32(0.0)
            for p in (w * rotated[t]).astype(np.float32):
                s = np.float32(s + p)
            plain[t, r] = s
    assert not np.array_equal(plain.view(np.uint32), v.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("bits", WIDTHS)
@pytest.mark.parametrize("group,rows,columns", [(64, 40, 100), (128, 300, 700), (256, 17, 2048), (128, 2048, 512)])
def test_gpu_float_path_bit_exact(bits, group, rows, columns):
    blob, cb, om = _matrix(rows, columns, group, bits, seed=bits * 3 + rows)
    m = rn.CodebookMatrix(blob, rows, columns, group, bits, cb)
    rng = np.random.default_rng(rows + bits)
    rotated = rng.standard_normal((5, m.padded)).astype(np.float32)
    for batch in (False, True):
        got = m.multiply_float_host(rotated, batch=batch)
        want = om.multiply_float(rotated, batch=batch)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (bits, group, batch)
    if bits in (1, 3):  # no integer levels: the ordinary entry points are the float path
        assert np.array_equal(m.multiply_batch_host(rotated[:1]).view(np.uint32),
                              om.multiply_float(rotated[:1]).view(np.uint32))
        assert np.array_equal(m.multiply_batch_host(rotated).view(np.uint32),
                              om.multiply_float(rotated, batch=True).view(np.uint32))
        assert np.array_equal(m.dequantise_row(rows - 1).view(np.uint32), om.dequantise_row(rows - 1).view(np.uint32))

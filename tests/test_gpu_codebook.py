"""Codebook-format products on the GPU against the oracle, bit for bit, through the C ABI."""
import numpy as np
import pytest

import oracle
import rustyneedle_amd as rn

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _pair(bits, group, rows, columns, seed):
    cb = rn.synthetic_codebook(group)
    blob = rn.synthetic_codebook_blob(rows, columns, group, bits, seed=seed)
    return (rn.CodebookMatrix(blob, rows, columns, group, bits, cb),
            oracle.OracleCodebookMatrix(blob, rows, columns, group, bits, cb))


SHAPES = [
    (2, 128, 1, 128),       # one row, one group
    (2, 128, 2048, 512),    # a layer product
    (2, 64, 37, 200),       # ragged rows, columns padded to the group
    (2, 256, 300, 1536),    # rows per block not a power of two
    (4, 128, 513, 512),
    (4, 64, 100, 130),
    (4, 256, 64, 4096),
    (5, 128, 129, 384),     # ternary crumbs
    (5, 64, 8, 64),
    (2, 128, 4, 40000),     # 626 chunks a row: 16 loads a lane, one row a block
    (4, 128, 3, 20000),
]


@pytest.mark.parametrize("bits,group,rows,columns", SHAPES)
def test_prepare_and_vector_product(bits, group, rows, columns):
    g, o = _pair(bits, group, rows, columns, seed=rows + columns)
    x = rn.synth_normal(5, "cbx", 1.0, (columns,))
    rotated = g.prepare_host(x)
    assert np.array_equal(_bits(rotated[0]), _bits(o.prepare(x)))
    y, acc = g.multiply_batch_host(rotated, with_acc=True)
    yo, acco = o.multiply_rotated(rotated, with_acc=True)
    assert np.array_equal(acc, acco)
    assert np.array_equal(_bits(y), _bits(yo))


@pytest.mark.parametrize("bits,group,rows,columns,count", [
    (2, 128, 512, 512, 3), (2, 128, 300, 512, 9), (4, 128, 130, 384, 17), (5, 256, 70, 1024, 8),
    (2, 64, 64, 4096, 5), (4, 64, 96, 2048, 12)])
def test_batch_product(bits, group, rows, columns, count):
    g, o = _pair(bits, group, rows, columns, seed=count)
    x = rn.synth_normal(6, "cbxb", 1.0, (count, columns))
    x[1] *= 1e-3  # a different scale per token
    rotated = g.prepare_host(x)
    assert np.array_equal(_bits(rotated), _bits(np.stack([o.prepare(v) for v in x])))
    y, acc = g.multiply_batch_host(rotated, with_acc=True)
    yo, acco = o.multiply_rotated(rotated, with_acc=True)
    assert np.array_equal(acc, acco)
    assert np.array_equal(_bits(y), _bits(yo))


def test_zero_and_sparse_inputs():
    g, o = _pair(2, 128, 96, 512, seed=1)
    x = np.zeros((2, 512), np.float32)
    x[1, 3] = -2.5  # one non-zero value: every other group has peak 0 and scale 1
    rotated = g.prepare_host(x)
    y, acc = g.multiply_batch_host(rotated, with_acc=True)
    yo, acco = o.multiply_rotated(rotated, with_acc=True)
    assert not y[0].any() and not acc[0].any()
    assert np.array_equal(acc, acco) and np.array_equal(_bits(y), _bits(yo))


@pytest.mark.parametrize("bits,group,columns", [(2, 128, 512), (4, 64, 200), (5, 256, 1024)])
def test_dequantise_row(bits, group, columns):
    g, o = _pair(bits, group, 9, columns, seed=2)
    for r in (0, 4, 8):
        assert np.array_equal(_bits(g.dequantise_row(r)), _bits(o.dequantise_row(r)))


def test_fused_products_share_the_rotated_input():
    pairs = [_pair(2, 128, rows, 512, seed=rows) for rows in (512, 128, 384)]
    x = rn.synth_normal(8, "cbf", 1.0, (512,))
    rotated = pairs[0][0].prepare_host(x)
    ys = rn.multiply_fused_host([g for g, _ in pairs], rotated[0])
    for (g, o), y in zip(pairs, ys):
        assert np.array_equal(_bits(y), _bits(o.multiply_rotated(rotated)[0]))



def test_matrix_from_an_archive_record():
    """QuantisedMatrix::from_archive: the record's blob, shape, group and bits, and
    the archive's codebook, give the same product as the blob given directly."""
    from cact_writer import write
    cb = rn.synthetic_codebook(128)
    blobs = {bits: rn.synthetic_codebook_blob(96, 300, 128, bits, seed=bits) for bits in (2, 4, 5)}
    data = write([(1, (8,), np.zeros(8, np.float16).tobytes(), 0, 0)] +
                 [(3, (96, 300), blobs[b].tobytes(), 128, b) for b in (2, 4, 5)], cb)
    a = rn.Archive(data=data)
    x = rn.synth_normal(4, "cbarch", 1.0, (300,))
    for index, bits in ((1, 2), (2, 4), (3, 5)):
        g = a.matrix(index)
        o = oracle.OracleCodebookMatrix(blobs[bits], 96, 300, 128, bits, cb)
        rotated = g.prepare_host(x)
        assert np.array_equal(_bits(g.multiply_batch_host(rotated)), _bits(o.multiply_rotated(rotated)))
        assert np.array_equal(_bits(g.dequantise_row(95)), _bits(o.dequantise_row(95)))

"""GPU parity of the gfx950 kernels against the oracle, through the C ABI.

The bar is bit-exact: integer accumulators, quantised codes and every float
(the kernels use the same operation order as the oracle).
"""
import numpy as np
import pytest

import oracle
import rustyneedle_amd as rn

pytestmark = pytest.mark.gpu
G = 32


def _matrix(rng, rows, cols):
    W = rng.integers(-127, 128, size=(rows, cols), dtype=np.int8)
    sW = rng.uniform(1e-3, 1e-2, size=(rows, cols // G)).astype(np.float32)
    return W, sW


def test_fast_exp_and_silu_bit_exact():
    rng = np.random.default_rng(1)
    x = np.concatenate([np.linspace(-100, 100, 20001, dtype=np.float32),
                        rng.standard_normal(5000).astype(np.float32) * 20,
                        np.array([0.0, -0.0, 87.0, -87.0, 88.0, -88.0, 1e-30], np.float32)])
    e = rn.fast_exp(x)
    s = rn.silu(x)
    assert np.array_equal(e.view(np.uint32), np.array([oracle.fast_exp(float(v)) for v in x], np.float32).view(np.uint32))
    assert np.array_equal(s.view(np.uint32), np.array([oracle.silu(float(v)) for v in x], np.float32).view(np.uint32))


@pytest.mark.parametrize("cols", [16, 512, 2048, 3000])
def test_quantise_bit_exact(cols):
    rng = np.random.default_rng(cols)
    x = (rng.standard_normal((9, cols)) * rng.uniform(0.1, 100, size=(9, 1))).astype(np.float32)
    x[3] = 0.0
    x[4, :7] = [0.5, 1.5, 2.5, -0.5, -1.5, 127.0, -127.0]
    x[4, 7:] = 0.0
    codes, scales = rn.quantise_int8(x)
    for t in range(9):
        c, s = oracle.quantise_int8(x[t])
        assert np.array_equal(codes[t], c), t
        assert scales[t] == s, t


@pytest.mark.parametrize("n", [8, 512, 2048])
def test_zero_centred_norm_bit_exact(n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((5, n)) * 9).astype(np.float32)
    g = (rng.standard_normal(n) * 0.1).astype(np.float32)
    out = rn.zero_centred_norm(x, g)
    for t in range(5):
        assert np.array_equal(out[t].view(np.uint32), oracle.zero_centred_norm(x[t], g).view(np.uint32))


@pytest.mark.parametrize("rows,cols,form", [
    (2048, 512, rn.FORM_PANEL),    # the single int8 matvec of the GEMV workload
    (2048, 512, rn.FORM_PLANE),
    (1536, 512, rn.FORM_PANEL),
    (512, 2048, rn.FORM_PANEL),
    (8192, 512, rn.FORM_PLANE),
    (100, 1024, rn.FORM_PANEL),    # ragged last block
    (7, 2048, rn.FORM_PLANE),
    (1, 512, rn.FORM_PANEL),
    (1152, 384, rn.FORM_PANEL),    # the d_model 384 products of the speech path
    (8192, 384, rn.FORM_PLANE),
    (384, 1536, rn.FORM_PANEL),
    (13, 384, rn.FORM_PANEL),
    (5, 1536, rn.FORM_PLANE),
])
def test_multiply_vector_bit_exact(rows, cols, form):
    rng = np.random.default_rng(rows * 7 + cols + form)
    W, sW = _matrix(rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    m = rn.QuantisedMatrix(W, sW, form)
    y, acc = m.multiply_vector_host(x, with_acc=True)
    yo, acco, _, _ = oracle.multiply(form, W, sW, x, with_acc=True)
    assert np.array_equal(acc, acco[0])
    assert np.array_equal(y.view(np.uint32), yo[0].view(np.uint32))


@pytest.mark.parametrize("rows", [2048, 1000])
@pytest.mark.parametrize("rows_per_block", [8, 16, 32])
def test_multiply_vector_rows_instances(rows, rows_per_block):
    """The product's 8-, 16- and 32-row kernel instances give the oracle's bits
    (the 8-row one is the instance a 2048 x 512 product runs)."""
    rng = np.random.default_rng(rows + rows_per_block)
    W, sW = _matrix(rng, rows, 512)
    x = rng.standard_normal(512).astype(np.float32)
    m = rn.QuantisedMatrix(W, sW)
    xd, yd = rn.DeviceBuffer.from_array(x), rn.DeviceBuffer(4 * rows)
    m.multiply_vector_rows(xd.ptr, yd.ptr, rows_per_block)
    rn.check(rn.lib.rn_stream_synchronize(None))
    y = yd.download(np.float32, (rows,))
    yo = oracle.multiply(0, W, sW, x)[0][0]
    assert np.array_equal(y.view(np.uint32), yo.view(np.uint32))
    with pytest.raises(rn.RnError):
        m.multiply_vector_rows(xd.ptr, yd.ptr, 12)


def test_multiply_vector_edge_inputs():
    rng = np.random.default_rng(5)
    W, sW = _matrix(rng, 256, 512)
    m = rn.QuantisedMatrix(W, sW)
    for x in (np.zeros(512, np.float32), np.full(512, -3.0, np.float32),
              np.eye(1, 512, 77, dtype=np.float32)[0] * 1e-30):
        y, acc = m.multiply_vector_host(x, with_acc=True)
        yo, acco, _, _ = oracle.multiply(0, W, sW, x, with_acc=True)
        assert np.array_equal(acc, acco[0]) and np.array_equal(y.view(np.uint32), yo[0].view(np.uint32))


@pytest.mark.parametrize("rows", [(512, 128, 128, 512), (37, 1000, 200), (3, 2048)])
def test_multiply_fused_matches_separate(rows):
    # each matrix is a grid row of one launch; a matrix with fewer blocks than
    # the widest leaves spare blocks, which must store nothing
    rng = np.random.default_rng(9)
    mats = [_matrix(rng, r, 512) for r in rows]
    x = rng.standard_normal(512).astype(np.float32)
    qm = [rn.QuantisedMatrix(W, sW) for W, sW in mats]
    ys = rn.multiply_fused_host(qm, x)
    for (W, sW), y in zip(mats, ys):
        yo = oracle.multiply(0, W, sW, x)[0][0]
        assert np.array_equal(y.view(np.uint32), yo.view(np.uint32))


@pytest.mark.parametrize("count,rows,cols,form", [
    (1, 512, 512, rn.FORM_PANEL),
    (7, 1536, 512, rn.FORM_PANEL),
    (64, 4096, 512, rn.FORM_PANEL),
    (64, 512, 2048, rn.FORM_PANEL),
    (256, 1536, 512, rn.FORM_PANEL),
    # the 256-token prefill shapes: fused gate/up, out and down
    (256, 4096, 512, rn.FORM_PANEL),
    (256, 512, 512, rn.FORM_PANEL),
    (256, 512, 2048, rn.FORM_PANEL),
    (65, 1000, 512, rn.FORM_PLANE),
    (3, 64, 1024, rn.FORM_PLANE),
    (100, 1152, 384, rn.FORM_PANEL),
    (33, 384, 1536, rn.FORM_PANEL),
    (17, 8192, 384, rn.FORM_PLANE),
    # grids of 256 blocks or more take the register-chain kernel: ragged token
    # and row tiles, a long K, the plane form
    (300, 1000, 512, rn.FORM_PANEL),
    (1500, 384, 1536, rn.FORM_PANEL),
    (600, 1000, 384, rn.FORM_PLANE),
])
def test_multiply_batch_mfma_bit_exact(count, rows, cols, form):
    rng = np.random.default_rng(count * 13 + rows + cols)
    W, sW = _matrix(rng, rows, cols)
    x = rng.standard_normal((count, cols)).astype(np.float32)
    m = rn.QuantisedMatrix(W, sW, form)
    y, acc = m.multiply_batch_host(x, with_acc=True)
    yo, acco, _, _ = oracle.multiply(form, W, sW, x, with_acc=True)
    assert np.array_equal(acc, acco)
    assert np.array_equal(y.view(np.uint32), yo.view(np.uint32))
    y2 = m.multiply_batch_host(x)  # the non-dumping kernel
    assert np.array_equal(y2.view(np.uint32), yo.view(np.uint32))


def test_batch_row_equals_vector():
    """A token's row of the MFMA product is the batch-1 product of that token."""
    rng = np.random.default_rng(17)
    W, sW = _matrix(rng, 1536, 512)
    x = rng.standard_normal((5, 512)).astype(np.float32)
    m = rn.QuantisedMatrix(W, sW)
    yb = m.multiply_batch_host(x)
    for t in range(5):
        assert np.array_equal(yb[t].view(np.uint32), m.multiply_vector_host(x[t]).view(np.uint32))


@pytest.mark.parametrize("lengths", [[1], [2, 15, 16, 17], [100, 1, 544, 33], [1024]])
def test_attend_heads_bit_exact(lengths):
    rng = np.random.default_rng(sum(lengths))
    count, stride = len(lengths), max(lengths)
    q = (rng.standard_normal((count, 64)) * 3).astype(np.float32)
    K = rng.standard_normal((count, stride, 64)).astype(np.float16)
    V = rng.standard_normal((count, stride, 64)).astype(np.float16)
    out = rn.attend_heads(q, K, V, np.array(lengths))
    for i, L in enumerate(lengths):
        ref = oracle.attend_head(q[i], K[i, :L], V[i, :L])
        assert np.array_equal(out[i].view(np.uint32), ref.view(np.uint32)), (i, L)


def test_attend_heads_rejects_bad_length():
    q = np.zeros((1, 64), np.float32)
    K = np.zeros((1, 4, 64), np.float16)
    with pytest.raises(rn.RnError):
        rn.attend_heads(q, K, K, np.array([5]))


def _near_boundary_rows(rng, count, cols):
    """Rows whose quotients by their own scale sit within a few ulps of
    half-integers: the inputs where a reciprocal-based quantiser could differ
    from the division."""
    rows = np.empty((count, cols), np.float32)
    for t in range(count):
        peak = np.float32(10.0 ** rng.uniform(-3, 3))
        s = np.float32(peak / np.float32(127))
        k = rng.integers(-127, 127, cols).astype(np.float32)
        v = ((k + np.float32(0.5)) * s).astype(np.float32)
        steps = rng.integers(-3, 4, cols)
        for u in range(1, 4):
            v = np.where(steps >= u, np.nextafter(v, np.float32(np.inf)), v)
            v = np.where(steps <= -u, np.nextafter(v, np.float32(-np.inf)), v)
        v[0] = peak
        rows[t] = np.clip(v, -peak, peak)
    return rows


def test_quantise_near_rounding_boundaries():
    rng = np.random.default_rng(41)
    x = _near_boundary_rows(rng, 16, 2048)
    codes, scales = rn.quantise_int8(x)
    for t in range(x.shape[0]):
        c, s = oracle.quantise_int8(x[t])
        assert scales[t] == s
        assert np.array_equal(codes[t], c), t


@pytest.mark.parametrize("cols", [512, 2048])
def test_products_quantise_near_rounding_boundaries(cols):
    """The matvec prologue and the batched row quantiser on the same inputs."""
    rng = np.random.default_rng(cols + 5)
    W, sW = _matrix(rng, 256, cols)
    x = _near_boundary_rows(rng, 8, cols)
    m = rn.QuantisedMatrix(W, sW)
    yo, acco, _, _ = oracle.multiply(rn.FORM_PANEL, W, sW, x, with_acc=True)
    yb, accb = m.multiply_batch_host(x, with_acc=True)
    assert np.array_equal(accb, acco)
    assert np.array_equal(yb.view(np.uint32), yo.view(np.uint32))
    for t in range(x.shape[0]):
        y, acc = m.multiply_vector_host(x[t], with_acc=True)
        assert np.array_equal(acc, acco[t])
        assert np.array_equal(y.view(np.uint32), yo[t].view(np.uint32))

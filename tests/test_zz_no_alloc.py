"""rn_matrix_multiply_batch_noalloc against rn_matrix_multiply_batch, through
the C ABI: bit-exact outputs (and int32 accumulators) on two calls in a row,
the second with fewer rows, so the fixed scratch keeps the first call's
contents while the second runs; sizes beyond the scratch are refused."""
import ctypes as C

import numpy as np
import pytest

import rustyneedle_amd as rn

pytestmark = pytest.mark.gpu

lib = rn.lib


def _run(entry, m, x, rows, acc_groups=None):
    count = x.shape[0]
    xd = rn.DeviceBuffer.from_array(x)
    yd = rn.DeviceBuffer(4 * count * rows)
    ad = rn.DeviceBuffer(4 * count * rows * acc_groups) if acc_groups else None
    rc = entry(m.handle, xd.ptr, count, yd.ptr, ad.ptr if ad else None, None)
    assert rc == rn.RN_OK, lib.rn_last_error()
    rn.check(lib.rn_stream_synchronize(None))
    y = yd.download(np.float32, (count, rows))
    acc = ad.download(np.int32, (count, rows, acc_groups)) if ad else None
    return y, acc


@pytest.mark.parametrize("rows,cols,form,counts", [
    (1536, 512, rn.FORM_PANEL, (256, 17)),
    (512, 2048, rn.FORM_PANEL, (2048, 64)),   # exactly the 4 MiB of codes, then fewer rows
    (1000, 384, rn.FORM_PLANE, (600, 3)),
])
def test_noalloc_equals_batch_twice(rows, cols, form, counts):
    rng = np.random.default_rng(rows + cols)
    W = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
    sW = rng.uniform(1e-3, 1e-2, (rows, cols // 32)).astype(np.float32)
    m = rn.QuantisedMatrix(W, sW, form)
    for count in counts:
        x = rng.standard_normal((count, cols)).astype(np.float32)
        ref, _ = _run(lib.rn_matrix_multiply_batch, m, x, rows)
        got, _ = _run(lib.rn_matrix_multiply_batch_noalloc, m, x, rows)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), count
    # with the int32 accumulator dump, a large call then a small one
    for count in (counts[0] // 2 or 1, 5):
        x = rng.standard_normal((count, cols)).astype(np.float32)
        ref, racc = _run(lib.rn_matrix_multiply_batch, m, x, rows, cols // 32)
        got, gacc = _run(lib.rn_matrix_multiply_batch_noalloc, m, x, rows, cols // 32)
        assert np.array_equal(gacc, racc)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_noalloc_refuses_sizes_beyond_the_scratch():
    W = np.ones((64, 2048), np.int8)
    sW = np.ones((64, 64), np.float32)
    m = rn.QuantisedMatrix(W, sW)
    # checked on the host before any device work: pointers are never touched
    fake = C.c_void_p(16)
    rc = lib.rn_matrix_multiply_batch_noalloc(m.handle, fake, 2049, fake, None, None)
    assert rc == rn.RN_ERR_ARGUMENT and b"scratch" in lib.rn_last_error()
    W2 = np.ones((64, 512), np.int8)
    m2 = rn.QuantisedMatrix(W2, np.ones((64, 16), np.float32))
    rc = lib.rn_matrix_multiply_batch_noalloc(m2.handle, fake, 4097, fake, None, None)
    assert rc == rn.RN_ERR_ARGUMENT and b"scratch" in lib.rn_last_error()

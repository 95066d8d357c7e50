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
    """The size check runs on the host before any device work. The buffers are
    real and large enough for the refused sizes, so a regression of the check
    would compute into them instead of writing out of bounds."""
    W = np.ones((64, 2048), np.int8)
    sW = np.ones((64, 64), np.float32)
    m = rn.QuantisedMatrix(W, sW)
    xd = rn.DeviceBuffer(4 * 4097 * 2048)
    yd = rn.DeviceBuffer(4 * 4097 * 64)
    rc = lib.rn_matrix_multiply_batch_noalloc(m.handle, xd.ptr, 2049, yd.ptr, None, None)
    assert rc == rn.RN_ERR_ARGUMENT and b"scratch" in lib.rn_last_error()
    W2 = np.ones((64, 512), np.int8)
    m2 = rn.QuantisedMatrix(W2, np.ones((64, 16), np.float32))
    rc = lib.rn_matrix_multiply_batch_noalloc(m2.handle, xd.ptr, 4097, yd.ptr, None, None)
    assert rc == rn.RN_ERR_ARGUMENT and b"scratch" in lib.rn_last_error()
    rn.check(lib.rn_stream_synchronize(None))


@pytest.mark.parametrize("bits", [2, 4, 3])
def test_noalloc_codebook_and_float_path(bits):
    """The branches that need no scratch: a 2- or 4-bit codebook matrix (the
    integer product, with its int32 group sums) and a 3-bit one (the float
    path's batch tile, which has no accumulators and refuses acc), each bit for
    bit against rn_matrix_multiply_batch on two calls, the second smaller."""
    rows, columns, group = 384, 512, 128
    cb = rn.synthetic_codebook(group)
    blob = rn.synthetic_codebook_blob(rows, columns, group, bits, name=f"noalloc.{bits}")
    m = rn.CodebookMatrix(blob, rows, columns, group, bits, cb)
    rng = np.random.default_rng(bits)
    groups = m.padded // group
    for count in (40, 7):
        x = rng.standard_normal((count, m.padded)).astype(np.float32)
        ref, _ = _run(lib.rn_matrix_multiply_batch, m, x, rows)
        got, _ = _run(lib.rn_matrix_multiply_batch_noalloc, m, x, rows)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (bits, count)
        if bits == 3:
            xd = rn.DeviceBuffer.from_array(x)
            yd = rn.DeviceBuffer(4 * count * rows)
            ad = rn.DeviceBuffer(4 * count * rows * groups)
            rc = lib.rn_matrix_multiply_batch_noalloc(m.handle, xd.ptr, count, yd.ptr, ad.ptr, None)
            assert rc == rn.RN_ERR_ARGUMENT and b"accumulators" in lib.rn_last_error()
        else:
            ref, racc = _run(lib.rn_matrix_multiply_batch, m, x, rows, groups)
            got, gacc = _run(lib.rn_matrix_multiply_batch_noalloc, m, x, rows, groups)
            assert np.array_equal(gacc, racc) and np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_noalloc_calls_on_two_streams_are_ordered():
    """Calls on two streams from two threads: each result equals the
    allocating entry point's, because the calls on one GPU are ordered (the
    second call's stream waits for the first call's kernels)."""
    import threading
    rows, cols = 1536, 512
    rng = np.random.default_rng(9)
    W = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
    sW = rng.uniform(1e-3, 1e-2, (rows, cols // 32)).astype(np.float32)
    m = rn.QuantisedMatrix(W, sW, rn.FORM_PANEL)
    xs = [rng.standard_normal((count, cols)).astype(np.float32) for count in (300, 301, 77, 256)]
    refs = [_run(lib.rn_matrix_multiply_batch, m, x, rows)[0] for x in xs]
    streams = []
    for _ in range(2):
        h = C.c_void_p()
        rn.check(lib.rn_stream_create(C.byref(h)))
        streams.append(h.value)
    outs = [None] * len(xs)
    bufs = [(rn.DeviceBuffer.from_array(x), rn.DeviceBuffer(4 * x.shape[0] * rows)) for x in xs]

    codes = []

    def work(k):
        for i in range(k, len(xs), 2):
            for _ in range(3):
                codes.append(lib.rn_matrix_multiply_batch_noalloc(m.handle, bufs[i][0].ptr, xs[i].shape[0],
                                                                  bufs[i][1].ptr, None, streams[k]))

    threads = [threading.Thread(target=work, args=(k,)) for k in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    for h in streams:
        rn.check(lib.rn_stream_synchronize(h))
    assert codes == [rn.RN_OK] * 3 * len(xs)
    for i, x in enumerate(xs):
        outs[i] = bufs[i][1].download(np.float32, (x.shape[0], rows))
        assert np.array_equal(outs[i].view(np.uint32), refs[i].view(np.uint32)), i
    for h in streams:
        rn.check(lib.rn_stream_destroy(h))

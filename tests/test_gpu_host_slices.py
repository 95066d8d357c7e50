"""The host-slice product entry points, called the way the reference-side
binding calls them: a matrix made from host codes and scales, then
multiply_vector / multiply_batch / prepare with plain host arrays for input
and output (QuantisedMatrix::multiply_vector(&self, &[f32], &mut [f32]),
crates/kernels/src/matrix.rs:155-165; multiply_batch, matrix.rs:330-389;
prepare_batch, matrix.rs:130-138). Results are bit-exact against the oracle,
and equal to the device-pointer entry points. Several threads share one
matrix, as the reference's Send + Sync matrix allows."""
import ctypes as C
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import oracle
import rustyneedle_amd as rn

pytestmark = pytest.mark.gpu

lib = rn.lib


def _u32(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _create_i8(codes, scales, form):
    h = C.c_void_p()
    rows, cols = codes.shape
    rc = lib.rn_matrix_create_i8(codes.ctypes.data, scales.ctypes.data, rows, cols, 32, form, C.byref(h))
    assert rc == rn.RN_OK, lib.rn_last_error()
    return h.value


@pytest.mark.parametrize("rows,cols,form", [(2048, 512, rn.FORM_PANEL), (1000, 2048, rn.FORM_PLANE),
                                            (64, 384, rn.FORM_PANEL)])
def test_vector_and_batch_from_host_slices(rows, cols, form):
    rng = np.random.default_rng(rows + cols)
    codes = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
    scales = rng.uniform(1e-3, 1e-2, (rows, cols // 32)).astype(np.float32)
    handle = _create_i8(codes, scales, form)
    try:
        x = rng.standard_normal(cols).astype(np.float32)
        y = np.full(rows, np.nan, dtype=np.float32)
        assert lib.rn_matrix_multiply_vector_host(handle, x.ctypes.data, y.ctypes.data) == rn.RN_OK
        ref = oracle.multiply(form, codes, scales, x)[0][0]
        assert np.array_equal(_u32(y), _u32(ref))
        for count in (1, 5, 64):
            xb = rng.standard_normal((count, cols)).astype(np.float32)
            yb = np.full((count, rows), np.nan, dtype=np.float32)
            assert lib.rn_matrix_multiply_batch_host(handle, xb.ctypes.data, count, yb.ctypes.data) == rn.RN_OK
            refb = oracle.multiply(form, codes, scales, xb)[0]
            assert np.array_equal(_u32(yb), _u32(refb)), count
        # a second, smaller call reuses the staging buffer
        y2 = np.empty(rows, dtype=np.float32)
        assert lib.rn_matrix_multiply_vector_host(handle, x.ctypes.data, y2.ctypes.data) == rn.RN_OK
        assert np.array_equal(_u32(y2), _u32(ref))
    finally:
        lib.rn_matrix_free(handle)


def test_host_slices_equal_device_pointers_and_threads_share_a_matrix():
    rng = np.random.default_rng(5)
    rows, cols = 1536, 512
    codes = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
    scales = rng.uniform(1e-3, 1e-2, (rows, cols // 32)).astype(np.float32)
    m = rn.QuantisedMatrix(codes, scales)
    xs = rng.standard_normal((16, cols)).astype(np.float32)
    dev = [m.multiply_vector_host(x) for x in xs]

    def call(i):
        y = np.empty(rows, dtype=np.float32)
        assert lib.rn_matrix_multiply_vector_host(m.handle, xs[i].ctypes.data, y.ctypes.data) == rn.RN_OK
        return y

    with ThreadPoolExecutor(4) as ex:
        got = list(ex.map(call, [i % 16 for i in range(64)]))
    for i, y in enumerate(got):
        assert np.array_equal(_u32(y), _u32(dev[i % 16])), i


def test_codebook_prepare_and_vector_from_host_slices():
    rows, columns, group, bits = 300, 700, 128, 2
    cb = rn.synthetic_codebook(group)
    blob = rn.synthetic_codebook_blob(rows, columns, group, bits, name="host_slices.cb")
    m = rn.CodebookMatrix(blob, rows, columns, group, bits, cb)
    om = oracle.OracleCodebookMatrix(blob, rows, columns, group, bits, cb)
    rng = np.random.default_rng(9)
    x = rng.standard_normal((3, columns)).astype(np.float32)
    rotated = np.empty((3, m.padded), dtype=np.float32)
    assert lib.rn_matrix_prepare_host(m.handle, x.ctypes.data, 3, rotated.ctypes.data) == rn.RN_OK
    assert np.array_equal(_u32(rotated), _u32(np.stack([om.prepare(r) for r in x])))
    y = np.empty(rows, dtype=np.float32)
    assert lib.rn_matrix_multiply_vector_host(m.handle, rotated[0].ctypes.data, y.ctypes.data) == rn.RN_OK
    assert np.array_equal(_u32(y), _u32(om.multiply_rotated(rotated[:1])[0]))
    yb = np.empty((3, rows), dtype=np.float32)
    assert lib.rn_matrix_multiply_batch_host(m.handle, rotated.ctypes.data, 3, yb.ctypes.data) == rn.RN_OK
    assert np.array_equal(_u32(yb), _u32(om.multiply_rotated(rotated)))

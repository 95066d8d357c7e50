"""f32::ln as the reference calls it: the C library's logf (the log-mel features,
crates/whistle/src/frontend.rs:96-99, of mel energies plus the 2^-24 floor).

Oracle pins (CPU): the oracle calls the C library's logf itself, so the pins
check what that function is: known values (log 1 = +0, log e, log 2, the special
inputs: 0 -> -inf, negatives and NaN -> NaN, +inf -> +inf, the smallest
subnormal); within one ulp of log in float64 rounded once to float32 on a dense
sample of positive floats from 1e-30 to 1e30, so a wrong table entry or a dropped
term fails.

GPU: the device's libm_logf against the C library's on every one of the 2^32
float bit patterns, bit for bit; it is the method of ARM's optimized-routines
logf that glibc builds (16 subintervals with a (1/c, log c) table, a cubic in
double), the log of the device's log-mel kernel."""
import numpy as np
import pytest

import oracle
import rustyneedle_amd as rn


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_known_values():
    x = np.array([1.0, np.e, 2.0, 0.5, 0.0, -0.0, np.inf, -1.0, -np.inf, 1e-45], np.float32)
    y = oracle.libm_log_array(x)
    assert _bits(y[0]) == 0  # +0
    assert y[1] == np.float32(np.log(np.float64(np.float32(np.e))))
    assert y[2] == np.float32(np.log(2.0)) and y[3] == -np.float32(np.log(2.0))
    assert y[4] == -np.inf and y[5] == -np.inf and y[6] == np.inf
    assert np.isnan(y[7]) and np.isnan(y[8])
    assert y[9] == np.float32(np.log(np.float64(np.float32(1e-45))))
    assert np.isnan(oracle.libm_log_array(np.array([np.nan], np.float32))[0])


def test_within_one_ulp_of_the_correctly_rounded_value():
    x = np.geomspace(1e-30, 1e30, 2_000_001, dtype=np.float64).astype(np.float32)
    got = oracle.libm_log_array(x)
    want = np.log(x.astype(np.float64)).astype(np.float32)
    diff = np.abs(_bits(got).astype(np.int64) - _bits(want).astype(np.int64))
    assert diff.max() <= 1


@pytest.mark.gpu
def test_device_logf_equals_the_c_library_on_every_float():
    chunk = 1 << 27
    for start in range(0, 1 << 32, chunk):
        x = np.arange(start, start + chunk, dtype=np.uint64).astype(np.uint32).view(np.float32)
        got = rn.libm_log(x)
        want = oracle.libm_log_array(x)
        same = (_bits(got) == _bits(want)) | (np.isnan(got) & np.isnan(want))
        assert same.all(), (start, x[~same][:4], got[~same][:4], want[~same][:4])

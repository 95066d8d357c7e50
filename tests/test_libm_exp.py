"""f32::exp as the reference calls it: the C library's expf (sigmoid, ops.rs:68-71;
sinkhorn_in_place, ops.rs:198-217; the probe heads' online softmax,
heads.rs:138-150; the attention and engram gates, attention.rs:147-149,
session.rs:177-187).

Oracle pins (CPU): the oracle calls the C library's expf itself, so the pins
check what that function is. Known values (exp(0) = 1, exp(1) rounded, the
special inputs and the overflow and underflow thresholds); against exp in
float64 rounded once to float32 on a dense sample (the correctly rounded value:
glibc's expf evaluates a cubic in double whose error, about 2^-34 relative,
moves it across a rounding boundary for roughly one input in 2000, so the two
are at most one ulp apart and rarely differ); two inputs where glibc 2.35 rounds
up past the correctly rounded value, which a correctly rounded expf would fail.

GPU: the device's libm_expf against the C library's on every one of the 2^32
float bit patterns, and sigmoid over it on a sample; bit for bit."""
import numpy as np
import pytest

import oracle
import rustyneedle_amd as rn


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_known_values():
    x = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 88.8, -104.0, 88.72283, -103.97], np.float32)
    y = oracle.libm_exp_array(x)
    assert y[0] == 1.0 and y[1] == 1.0
    assert y[2] == np.float32(np.exp(np.float64(1.0))) and y[3] == np.float32(np.exp(np.float64(-1.0)))
    assert y[4] == np.inf and y[5] == 0.0 and y[6] == np.inf and y[7] == 0.0
    assert np.isfinite(y[8]) and y[9] > 0.0
    assert np.isnan(oracle.libm_exp_array(np.array([np.nan], np.float32))[0])


def test_within_one_ulp_of_the_correctly_rounded_value():
    x = np.linspace(-103.0, 88.0, 2_000_001, dtype=np.float32)
    got = oracle.libm_exp_array(x)
    want = np.exp(x.astype(np.float64)).astype(np.float32)
    diff = np.abs(_bits(got).astype(np.int64) - _bits(want).astype(np.int64))
    assert diff.max() <= 1
    assert 0 < np.count_nonzero(diff) <= x.size // 1000


def test_glibc_rounding_of_two_hard_cases():
    x = np.array([float.fromhex("0x1.04845ep+5"), float.fromhex("-0x1.f8cbb2p+5")], np.float32)
    got = oracle.libm_exp_array(x)
    assert [float(v).hex() for v in got] == ["0x1.f93e380000000p+46", "0x1.f453260000000p-92"]
    # one ulp above the correctly rounded values
    want = np.exp(x.astype(np.float64)).astype(np.float32)
    assert list(_bits(got) - _bits(want)) == [1, 1]


def test_sigmoid_is_one_over_one_plus_exp():
    x = np.linspace(-30, 30, 10001, dtype=np.float32)
    s = oracle.libm_exp_array(x, sigmoid=True)
    e = oracle.libm_exp_array(-x)
    assert np.array_equal(_bits(s), _bits(np.float32(1.0) / (np.float32(1.0) + e)))


@pytest.mark.gpu
def test_device_expf_equals_the_c_library_on_every_float():
    chunk = 1 << 27
    for start in range(0, 1 << 32, chunk):
        x = np.arange(start, start + chunk, dtype=np.uint64).astype(np.uint32).view(np.float32)
        got = rn.libm_exp(x)
        want = oracle.libm_exp_array(x)
        same = (_bits(got) == _bits(want)) | (np.isnan(got) & np.isnan(want))
        assert same.all(), (start, x[~same][:4], got[~same][:4], want[~same][:4])


@pytest.mark.gpu
def test_device_sigmoid_bit_exact():
    rng = np.random.default_rng(4)
    x = np.concatenate([np.linspace(-120, 120, 400001, dtype=np.float32),
                        (rng.standard_normal(200000) * 8).astype(np.float32),
                        np.array([0.0, -0.0, np.inf, -np.inf], np.float32)])
    assert np.array_equal(_bits(rn.sigmoid(x)), _bits(oracle.libm_exp_array(x, sigmoid=True)))

"""The reciprocal of the fused Needle 3 step's Sinkhorn normalisation
(sinkhorn_in_place, crates/kernels/src/ops.rs:198-217: `1.0 / total.max(
f32::MIN_POSITIVE)`), computed on the device as v_rcp_f32 and one Newton step
with fused multiply-adds instead of a division.

The divisor there is at least f32::MIN_POSITIVE (2^-126) and at most the lane
count (a row or column of exponentials of values no larger than the row's
peak, then of normalised ones), so the range the kernel relies on is
[2^-126, 2^126): every float of it is checked against the IEEE quotient.

CPU: the expected values are numpy's float32 division; they are checked here
against the float64 quotient rounded once to float32 (exact: 53 >= 2 * 24 + 2
bits, so the double rounding is innocuous) on a dense sample, and on powers of
two, where the reciprocal is exact."""
import numpy as np
import pytest

import rustyneedle_amd as rn

LO, HI = 0x00800000, 0x7E800000  # [2^-126, 2^126) as float bits


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_expected_values_are_correctly_rounded():
    rng = np.random.default_rng(7)
    b = rng.integers(LO, HI, 4_000_000, dtype=np.uint64).astype(np.uint32)
    x = b.view(np.float32)
    want = np.float32(1.0) / x
    via64 = (1.0 / x.astype(np.float64)).astype(np.float32)
    assert np.array_equal(_bits(want), _bits(via64))
    p = np.ldexp(np.float32(1.0), np.arange(-126, 126)).astype(np.float32)
    assert np.array_equal(np.float32(1.0) / p, np.ldexp(np.float32(1.0), -np.arange(-126, 126)).astype(np.float32))


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_device_reciprocal_equals_the_division_on_every_float_of_its_range():
    chunk = 1 << 27
    for start in range(LO, HI, chunk):
        stop = min(start + chunk, HI)
        x = np.arange(start, stop, dtype=np.uint32).view(np.float32)
        got = rn.reciprocal(x)
        want = np.float32(1.0) / x
        same = _bits(got) == _bits(want)
        assert same.all(), (hex(start), x[~same][:4], got[~same][:4], want[~same][:4])

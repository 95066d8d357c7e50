"""The speech front end on the GPU against the oracle. The FFT, power spectrum,
mel sums and normalisation follow the reference's float order; the log is the
device logf where the reference (and the oracle) call the host libm's logf, so
the bar is a tolerance: |gpu - oracle| <= 5e-5 (1 + |oracle|) on the normalised
features and 1e-5 relative on the spread (measured: at most 1.4e-5 (1 + |x|) over
a 30 s input, where a one-ulp difference of the log in most frames moves every
mel's mean and scale)."""
import numpy as np
import pytest

import oracle
import rustyneedle_amd as rn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,mels,fft,window,hop", [(480000, 80, 512, 400, 160), (16000, 80, 512, 400, 160),
                                                   (1000, 40, 256, 200, 100), (100, 16, 64, 48, 32),
                                                   (20, 16, 64, 48, 32), (0, 8, 32, 32, 16)])
def test_log_mel_matches_the_oracle(n, mels, fft, window, hop):
    rng = np.random.default_rng(n)
    x = (rng.normal(0, 0.1, n) + 0.3 * np.sin(np.arange(n) * 0.05)).astype(np.float32)
    w = rn.synthetic_mel_filters(mels, fft)
    f = rn.Frontend(mels, fft, window, hop, w)
    got, valid, spread = f.log_mel(x)
    want, vo, so = oracle.log_mel(x, mels, fft, window, hop, w)
    assert got.shape == want.shape and valid == vo
    assert np.all(np.abs(got - want) <= 5e-5 * (1.0 + np.abs(want)))
    assert abs(spread - so) <= 1e-5 * abs(so)
    assert not got[valid:].any()


def test_arguments():
    w = rn.synthetic_mel_filters(16, 64)
    with pytest.raises(rn.RnError):
        rn.Frontend(16, 48, 48, 16, np.zeros((25, 16), np.float32))  # not a power of two

"""The speech front end on the GPU against the oracle, bit for bit. The FFT,
power spectrum, mel sums and normalisation follow the reference's float order,
and the log is the device restatement of the C library's logf that the
reference (and the oracle) call (equal to it on every float input,
tests/test_libm_log.py). Whistle::encode from samples (the features handed to
the stem on the device) against the encode of the oracle's features."""
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
    assert np.array_equal(got.view(np.uint32), np.ascontiguousarray(want, np.float32).view(np.uint32))
    assert np.float32(spread).view(np.uint32) == np.float32(so).view(np.uint32)
    assert not got[valid:].any()


@pytest.mark.parametrize("frames,layers", [(3000, 6), (64, 2)])
def test_encode_from_samples_hands_the_features_over_on_the_device(frames, layers):
    """Whistle::encode (lib.rs:155-161) from samples: log-mel on the device, the
    stem reading the features in place; equal bit for bit to the encode of the
    oracle's log-mel features (whose encode is pinned to the oracle in
    test_gpu_whistle.py), and the spread to the oracle's."""
    cfg = dict(rn.WHISTLE)
    cfg.update(frames=frames, enc_layers=layers)
    hop, fft, window = 160, 512, 400
    rng = np.random.default_rng(frames)
    n = frames * hop
    x = (rng.normal(0, 0.1, n) + 0.3 * np.sin(np.arange(n) * 0.05)).astype(np.float32)
    w = rn.synthetic_mel_filters(cfg["mels"], fft)
    f = rn.Frontend(cfg["mels"], fft, window, hop, w)
    g = rn.Whistle(cfg, seed=5)
    want_mel, valid, so = oracle.log_mel(x, cfg["mels"], fft, window, hop, w)
    assert valid == frames
    ref = g.encode(np.ascontiguousarray(want_mel[:frames], np.float32))
    got, spread = g.encode_samples(f, x)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert np.float32(spread).view(np.uint32) == np.float32(so).view(np.uint32)
    with pytest.raises(rn.RnError):
        g.encode_samples(f, x[:-hop])  # one frame short of the model's frames


def test_arguments():
    w = rn.synthetic_mel_filters(16, 64)
    with pytest.raises(rn.RnError):
        rn.Frontend(16, 48, 48, 16, np.zeros((25, 16), np.float32))  # not a power of two

"""The speech front end's oracle (frontend.rs) pinned by closed forms and a
float64 restatement with numpy's FFT (the reference has no front-end tests)."""
import numpy as np

import oracle
import rustyneedle_amd as rn


def test_tables_are_the_hann_window_and_the_roots_of_unity():
    win, tc, ts = oracle.frontend_tables(512, 400)
    n = np.arange(400)
    assert np.max(np.abs(win - (0.5 - 0.5 * np.cos(2 * np.pi * n / 399)))) < 1e-6
    k = np.arange(256)
    assert np.max(np.abs(tc - np.cos(2 * np.pi * k / 512))) < 1e-6
    assert np.max(np.abs(ts + np.sin(2 * np.pi * k / 512))) < 1e-6


def test_power_spectrum_against_numpy_fft():
    rng = np.random.default_rng(2)
    for size in (8, 64, 512, 1024):
        re = rng.normal(0, 1, size).astype(np.float32)
        im = rng.normal(0, 1, size).astype(np.float32)
        got = oracle.power_spectrum(re, im)
        z = np.fft.fft(re.astype(np.float64) + 1j * im.astype(np.float64))
        want = np.abs(z[:size // 2 + 1]) ** 2
        assert np.max(np.abs(got - want)) < 1e-4 * want.max()


def test_a_tone_peaks_at_its_bin():
    t = np.arange(512)
    x = np.cos(2 * np.pi * 37 * t / 512).astype(np.float32)
    p = oracle.power_spectrum(x, np.zeros(512, np.float32))
    assert int(np.argmax(p)) == 37 and abs(p[37] - 256.0 ** 2) < 1.0


def _float64_log_mel(x, mels, fft, window, hop, w):
    frames, valid, half = x.size // hop + 1, x.size // hop, window // 2
    win = 0.5 - 0.5 * np.cos(2 * np.pi * np.arange(window) / (window - 1))
    data = np.zeros((frames, mels))
    for f in range(frames):
        buf = np.zeros(fft)
        for p in range(min(window, fft)):
            s = f * hop + p - half
            if 0 <= s < x.size:
                buf[p] = x[s] * win[p]
        power = np.abs(np.fft.fft(buf)[:fft // 2 + 1]) ** 2
        data[f] = np.log(power @ w.astype(np.float64) + 5.9604645e-8)
    v = data[:valid]
    spread = np.mean(np.std(v, axis=0, ddof=1)) if valid >= 2 else 0.0
    mean, std = v.mean(axis=0), v.std(axis=0, ddof=1 if valid > 1 else 0)
    out = np.where(np.arange(frames)[:, None] < valid, (data - mean) / (std + 1e-5), 0.0)
    return out, valid, spread


def test_log_mel_against_float64():
    rng = np.random.default_rng(4)
    w = rn.synthetic_mel_filters(80, 512)
    x = (rng.normal(0, 0.1, 16000) + 0.3 * np.sin(np.arange(16000) * 0.05)).astype(np.float32)
    got, valid, spread = oracle.log_mel(x, 80, 512, 400, 160, w)
    want, vw, sw = _float64_log_mel(x, 80, 512, 400, 160, w)
    assert got.shape == (101, 80) and valid == vw == 100
    assert np.max(np.abs(got - want)) < 2e-3
    assert abs(spread - sw) < 1e-4 * sw
    assert not got[100].any()                                   # past the valid frames
    assert np.max(np.abs(got[:100].mean(axis=0))) < 1e-4        # normalised columns
    assert np.max(np.abs(got[:100].std(axis=0, ddof=1) - 1.0)) < 1e-3


def test_silence_and_short_inputs():
    w = rn.synthetic_mel_filters(16, 64)
    got, valid, spread = oracle.log_mel(np.zeros(640, np.float32), 16, 64, 48, 32, w)
    # log(FLOOR) in every slot: only the float rounding of the mean deviates
    assert valid == 20 and spread < 1e-5
    assert np.array_equal(got[:20], np.broadcast_to(got[0], (20, 16))) and not got[20].any()
    got, valid, spread = oracle.log_mel(np.ones(20, np.float32), 16, 64, 48, 32, w)
    assert valid == 0 and spread == 0.0 and got.shape == (1, 16) and not got.any()

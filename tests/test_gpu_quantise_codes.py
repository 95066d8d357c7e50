"""The int8 code of a quotient on the device (code_of_quotient in
rustyneedle_amd/csrc/rn_device.hpp: v_rndne_f32, the saturating v_cvt_i32_f32,
then a clamp to [-128, 127]) against the rule of ops.rs:112-118 (round half
to even, clamp), for every float32 of [-127, 127].

A row whose peak is 127 has the scale 127 / 127 = 1 exactly, so each of its
elements is its own quotient; rn_quantise_int8 (one block a row) then gives
the code of every element. The expected codes are numpy's rint and clip."""
import numpy as np
import pytest

import rustyneedle_amd as rn

TOP = 0x42FE0000  # 127.0f
COLS = 4096       # column 0 holds the row's peak, 127


def _rows(vals: np.ndarray) -> np.ndarray:
    body = np.zeros(-(-vals.size // (COLS - 1)) * (COLS - 1), np.float32)
    body[:vals.size] = vals
    body = body.reshape(-1, COLS - 1)
    return np.concatenate([np.full((body.shape[0], 1), 127.0, np.float32), body], axis=1)


def test_rows_put_the_peak_first():
    x = _rows(np.array([1.5, -2.5, 0.25], np.float32))
    assert x.shape == (1, COLS) and x[0, 0] == 127.0 and list(x[0, 1:4]) == [1.5, -2.5, 0.25]


@pytest.mark.gpu
@pytest.mark.timeout(900)
def test_device_code_of_every_quotient_in_the_int8_range():
    chunk = (1 << 26) // (COLS - 1) * (COLS - 1)
    for sign in (0, 0x80000000):
        for start in range(0, TOP + 1, chunk):
            stop = min(start + chunk, TOP + 1)
            vals = (np.arange(start, stop, dtype=np.uint32) | np.uint32(sign)).view(np.float32)
            codes, scales = rn.quantise_int8(_rows(vals))
            assert (scales == np.float32(1.0)).all()
            got = codes[:, 1:].reshape(-1)[:vals.size]
            want = np.clip(np.rint(vals), -128, 127).astype(np.int8)
            same = got == want
            assert same.all(), (hex(start | sign), vals[~same][:4], got[~same][:4], want[~same][:4])

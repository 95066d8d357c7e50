"""Pins of the oracle's scalar primitives (crates/kernels/src/ops.rs) against the
reference's own known answers and against the mathematics.

Each check is chosen so that a plausible slip in the oracle fails it: a wrong
rounding rule, a dropped clamp, a wrong epsilon, a swapped rotary operand, a
different summation order, a last-index tie rule.
"""
import math

import numpy as np
import pytest

import oracle


# ---- fast_exp / softmax: crates/kernels/tests/softmax.rs:3-28 ------------------------

def test_fast_exp_reference_bound():
    """softmax.rs:4-14: <5e-6 relative on [-40, 5] in steps of 0.013, exp(0)=1, tiny at -200."""
    x = np.float32(-40.0)
    worst = 0.0
    while x <= 5.0:
        exact = math.exp(float(x))
        worst = max(worst, abs((oracle.fast_exp(float(x)) - exact) / exact))
        x = np.float32(x + np.float32(0.013))
    assert worst < 5e-6
    assert oracle.fast_exp(0.0) == 1.0
    v = oracle.fast_exp(-200.0)
    assert 0.0 <= v < 1e-30


def test_fast_exp_rounds_half_away_from_zero():
    """ops.rs:85 uses f32::round (ties away from zero): x*log2(e) = -0.5 must take
    whole = -1, fraction = +0.5; round-half-even would give whole = 0, fraction = -0.5,
    and a value that differs in the last bits."""
    x = np.float32(-0.5) / np.float32(1.4426950408889634)
    assert np.float32(x) * np.float32(1.4426950408889634) == np.float32(-0.5)
    whole = -1.0
    f = np.float32(0.5)
    c = [np.float32(v) for v in (0.6931471805599453, 0.2402265, 0.05550411, 0.009618129, 0.0013333558)]
    p = np.float32(1) + f * (c[0] + f * (c[1] + f * (c[2] + f * (c[3] + f * c[4]))))
    assert oracle.fast_exp(float(x)) == float(p * np.float32(2.0 ** whole))


def test_softmax_reference_values():
    """softmax.rs:18-27."""
    logits = np.array([3.1, -2.0, 0.5, 7.25, 7.2, -11.0], dtype=np.float32)
    p = oracle.softmax(logits)
    peak = float(logits.max())
    e = np.exp(logits.astype(np.float64) - peak)
    exact = e / e.sum()
    assert np.all(np.abs(p - exact) < 1e-6)
    assert abs(float(p.sum()) - 1.0) < 1e-6


def test_silu_uses_fast_exp():
    """ops.rs:73-76: silu(x) = x / (1 + fast_exp(-x)) exactly."""
    for v in (-30.0, -3.5, -1e-3, 0.0, 0.7, 2.0, 25.0):
        expect = np.float32(v) / (np.float32(1.0) + np.float32(oracle.fast_exp(-v)))
        assert oracle.silu(v) == float(expect)


# ---- quantisation: ops.rs:103-125 ------------------------------------------------------

def test_int8_scale_zero_vector_is_one():
    assert oracle.int8_scale(np.zeros(32, np.float32)) == 1.0
    codes, scale = oracle.quantise_int8(np.zeros(16, np.float32))
    assert scale == 1.0 and not codes.any()


def test_quantise_ties_round_to_even():
    """round_ties_even: with peak 127 the scale is exactly 1 and x/1 = x."""
    x = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.49, -126.5], dtype=np.float32)
    codes, scale = oracle.quantise_int8(x)
    assert scale == 1.0
    assert codes.tolist() == [127, 0, 2, 2, 0, -2, -2, 3, -126]


def test_quantise_peak_maps_to_127_and_matches_numpy():
    rng = np.random.default_rng(3)
    for n in (1, 7, 512, 2048):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        codes, scale = oracle.quantise_int8(x)
        peak = np.float32(np.abs(x).max())
        assert scale == np.float32(peak / np.float32(127.0))
        expect = np.clip(np.rint(x / scale), -128, 127).astype(np.int8)
        assert np.array_equal(codes, expect)
        assert np.abs(codes).max() == 127


def test_fake_quantise_is_codes_times_scale():
    x = np.random.default_rng(4).standard_normal(300).astype(np.float32)
    codes, scale = oracle.quantise_int8(x)
    assert np.array_equal(oracle.fake_quantise_int8(x), codes.astype(np.float32) * scale)


# ---- RMSNorm: ops.rs:7-17, 44-50 --------------------------------------------------------

def test_sum_of_squares_order_is_eight_strided_lanes():
    """The value of ops.rs:7-17 for 512 inputs, restated with numpy float32 lanes; a
    plain left-to-right sum gives a different float on this input."""
    x = np.random.default_rng(5).standard_normal(512).astype(np.float32) * np.float32(7.3)
    lanes = np.zeros(8, np.float32)
    for c in range(64):
        lanes = lanes + x[8 * c:8 * c + 8] * x[8 * c:8 * c + 8]
    total = np.float32(0)
    for j in range(8):
        total = np.float32(total + lanes[j])
    assert oracle.sum_of_squares(x) == float(total)
    naive = np.float32(0)
    for v in x:
        naive = np.float32(naive + v * v)
    assert float(naive) != float(total)
    assert abs(oracle.sum_of_squares(x) - float(np.sum(x.astype(np.float64) ** 2))) < 1e-4 * float(total)


def test_zero_centred_norm_against_float64():
    rng = np.random.default_rng(6)
    x = rng.standard_normal(512).astype(np.float32) * 5
    g = rng.standard_normal(512).astype(np.float32) * 0.1
    out = oracle.zero_centred_norm(x, g)
    x64 = x.astype(np.float64)
    ref = (1.0 + g.astype(np.float64)) * x64 / np.sqrt(np.mean(x64 ** 2) + 1e-6)
    assert np.max(np.abs(out - ref) / np.abs(ref).max()) < 2e-6
    # eps matters for a near-zero row: mean square 1e-12 -> inverse ~ 1/sqrt(1e-6) = 1000
    tiny = np.full(512, 1e-6, np.float32)
    assert abs(oracle.zero_centred_norm(tiny, np.zeros(512, np.float32))[0] - 1e-6 / math.sqrt(1e-12 + 1e-6)) < 1e-9


# ---- rotary: ops.rs:127-141 --------------------------------------------------------------

def test_rotary_frequencies_closed_form():
    f = oracle.rotary_frequencies(64, 10000.0)
    ref = 1.0 / 10000.0 ** (2.0 * np.arange(32) / 64.0)
    assert np.max(np.abs(f - ref) / ref) < 1e-6
    assert f[0] == 1.0


def test_rotary_identity_at_zero_and_norm_preserving():
    cos, sin = oracle.rotary_table(64, 10000.0, 300)
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    h = np.random.default_rng(8).standard_normal(64).astype(np.float32)
    assert np.array_equal(oracle.apply_rotary(h, cos[0], sin[0]), h)
    for pos in (1, 17, 255, 299):
        r = oracle.apply_rotary(h, cos[pos], sin[pos])
        assert abs(np.linalg.norm(r.astype(np.float64)) - np.linalg.norm(h.astype(np.float64))) < 1e-5
        # pairs (i, i+32) rotate by +angle: a' = a cos - b sin, b' = b cos + a sin
        ang = pos * (1.0 / 10000.0 ** (2.0 * np.arange(32) / 64.0))
        a, b = h[:32].astype(np.float64), h[32:].astype(np.float64)
        assert np.allclose(r[:32], a * np.cos(ang) - b * np.sin(ang), atol=2e-4)
        assert np.allclose(r[32:], b * np.cos(ang) + a * np.sin(ang), atol=2e-4)


# ---- fp16 ------------------------------------------------------------------------------

def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    finite = ~np.isnan(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[~finite]))


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(9)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32),
        (rng.standard_normal(5000) * 1e-5).astype(np.float32),   # subnormal halves
        (rng.standard_normal(2000) * 7e4).astype(np.float32),    # overflow to inf
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 2.0 ** -25, 2.0 ** -24, 1.5 * 2.0 ** -25,
                  1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], dtype=np.float32),
    ])
    ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)


# ---- argmax: generator.rs:257-265 --------------------------------------------------------

def test_argmax_first_index_of_strict_max():
    assert oracle.argmax([1.0, 3.0, 3.0, 2.0]) == 1
    assert oracle.argmax([5.0, 5.0]) == 0
    assert oracle.argmax([-0.0, 0.0]) == 0
    assert oracle.argmax([-np.inf, -np.inf, -1.0]) == 2


def test_argmax_nan_rules():
    nan = float("nan")
    assert oracle.argmax([nan, 1.0, 2.0]) == 0          # a NaN at 0 is never displaced
    assert oracle.argmax([1.0, nan, 3.0, nan]) == 2     # other NaNs never win
    assert oracle.argmax([-1.0, nan, nan]) == 0

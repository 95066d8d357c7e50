"""The constrained choice's oracle (generator.rs:147-194) pinned by known answers
and closed forms (the reference has no tests for these functions)."""
import math

import numpy as np

import oracle


def test_argmax_allowed_rules():
    v = np.array([1.0, 3.0, 2.0, 3.0, 5.0], np.float32)
    assert oracle.argmax_allowed(v, [1, 0, 1, 1, 0]) == 3        # largest allowed
    assert oracle.argmax_allowed(v, [0, 1, 0, 1, 0]) == 1        # ties: the first index
    assert oracle.argmax_allowed(v, [0, 0, 0, 0, 0]) == -1       # None
    n = np.array([np.nan, 1.0, 2.0], np.float32)
    assert oracle.argmax_allowed(n, [1, 1, 1]) == 0              # a NaN first allowed value wins
    assert oracle.argmax_allowed(n, [0, 1, 1]) == 2
    m = np.array([1.0, np.nan, 0.5], np.float32)
    assert oracle.argmax_allowed(m, [1, 1, 1]) == 0              # a later NaN never wins
    z = np.array([-0.0, 0.0, -np.inf], np.float32)
    assert oracle.argmax_allowed(z, [1, 1, 1]) == 0              # -0 and +0 are equal
    assert oracle.argmax_allowed(np.full(3, -np.inf, np.float32), [0, 1, 1]) == 1


def test_choose_falls_back_to_argmax():
    v = np.array([1.0, 3.0, 2.0], np.float32)
    assert oracle.choose_allowed(v, [0, 0, 0])[0] == 1


def test_statistics_closed_forms():
    rng = np.random.default_rng(3)
    v = rng.normal(0, 3, 8192).astype(np.float32)
    everything = np.ones(v.size, np.uint8)
    t = int(np.argmax(v))
    p, m = oracle.allowed_statistics(v, everything, t)
    assert m == np.float32(1.0)                                  # same terms, same order
    e = np.exp(v.astype(np.float64) - v.max())
    assert abs(p - 1.0 / e.sum()) < 1e-5 * (1.0 / e.sum())
    one = np.zeros(v.size, np.uint8)
    one[17] = 1
    p, m = oracle.allowed_statistics(v, one, 17)
    assert p == np.float32(1.0)                                  # fast_exp(0) / fast_exp(0)
    assert abs(m - math.exp(v[17] - v.max()) / e.sum()) < 1e-5 * m
    half = (rng.random(v.size) < 0.5).astype(np.uint8)
    t = oracle.argmax_allowed(v, half)
    p, m = oracle.allowed_statistics(v, half, t)
    ea = np.exp(v.astype(np.float64)[half == 1] - v[half == 1].max())
    assert abs(p - 1.0 / ea.sum()) < 1e-5 * p
    assert abs(m - (e[half == 1].sum() / e.sum())) < 1e-5 * m

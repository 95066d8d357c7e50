"""kronecker_apply (ops.rs:166-297) for 32 x 32 factors: the oracle against the
reference's own test (crates/kernels/tests/kronecker.rs: float64 reference,
1e-4 relative, on its deterministic inputs) and exact-rational fused
multiply-adds; the GPU bit for bit against the oracle."""
from fractions import Fraction

import numpy as np
import pytest

import oracle
import rustyneedle_amd as rn


def make(seed: int) -> np.ndarray:  # kronecker.rs:19
    i = np.arange(1024)
    return ((((i * 7919 + seed * 104729) % 2003).astype(np.float32) - 1000.0) / 500.0).astype(np.float32)


def test_matches_the_double_precision_reference():
    x, l, r = make(1), make(2), make(3)
    got = oracle.kronecker_apply_32(x, l, r)
    X, L, R = (a.astype(np.float64).reshape(32, 32) for a in (x, l, r))
    want = (L.T @ (X @ R)).reshape(-1)
    assert np.max(np.abs(want - got) / (1.0 + np.abs(want))) < 1e-4


def _round_f32(fr):
    x = np.float32(float(fr))
    best = x
    for cand in (np.nextafter(x, np.float32(-np.inf)), np.nextafter(x, np.float32(np.inf))):
        d_best, d_cand = abs(Fraction(float(best)) - fr), abs(Fraction(float(cand)) - fr)
        if d_cand < d_best or (d_cand == d_best and (int(cand.view(np.uint32)) & 1) == 0):
            best = cand
    return np.float32(best)


def test_fused_multiply_adds_in_index_order():
    x, l, r = make(4), make(5), make(6)
    got = oracle.kronecker_apply_32(x, l, r).reshape(32, 32)
    X, L, R = (a.reshape(32, 32) for a in (x, l, r))
    mixed = np.zeros((32, 32), np.float32)
    for i in range(32):
        for c in range(32):
            acc = np.float32(0)
            for j in range(32):
                acc = _round_f32(Fraction(float(R[j, c])) * Fraction(float(X[i, j])) + Fraction(float(acc)))
            mixed[i, c] = acc
    for k in (0, 7, 31):
        for c in (0, 13, 31):
            acc = np.float32(0)
            for i in range(32):
                acc = _round_f32(Fraction(float(mixed[i, c])) * Fraction(float(L[i, k])) + Fraction(float(acc)))
            assert got[k, c] == acc


@pytest.mark.gpu
def test_gpu_matches_the_oracle():
    rng = np.random.default_rng(9)
    xs = rng.normal(0, 1, (5, 1024)).astype(np.float32)
    l, r = rng.normal(0, 0.2, 1024).astype(np.float32), rng.normal(0, 0.2, 1024).astype(np.float32)
    got = rn.kronecker_apply(np.vstack([make(1)[None], xs]), l, r)
    for t, x in enumerate(np.vstack([make(1)[None], xs])):
        assert np.array_equal(got[t].view(np.uint32), oracle.kronecker_apply_32(x, l, r).view(np.uint32))
    with pytest.raises(rn.RnError):
        rn.check(rn.lib.rn_kronecker_apply(1, 1, 16, 1, 32, 1, 1, None))

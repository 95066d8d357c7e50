"""Pins of the oracle's quantised products and attention.

Integer accumulators are compared exactly with an int64 matrix product (a
different algorithm: numpy matmul over widened codes). Float results are
compared with float64 closed forms within stated tolerances, plus exact known
answers where the mathematics fixes the float result.
"""
from fractions import Fraction

import numpy as np
import pytest

import oracle

G = 32


def _matrix(rng, rows, cols):
    W = rng.integers(-127, 128, size=(rows, cols), dtype=np.int8)
    sW = rng.uniform(1e-3, 1e-2, size=(rows, cols // G)).astype(np.float32)
    return W, sW


@pytest.mark.parametrize("rows,cols,count", [(2048, 512, 1), (96, 2048, 3), (130, 1024, 5)])
def test_accumulators_equal_int64_matmul(rows, cols, count):
    rng = np.random.default_rng(rows + cols)
    W, sW = _matrix(rng, rows, cols)
    xq = rng.integers(-128, 128, size=(count, cols), dtype=np.int8)
    sx = rng.uniform(0.01, 0.05, size=count).astype(np.float32)
    y, acc = oracle.product(oracle.FORM_PANEL, W, sW, xq, sx, with_acc=True)
    ref = np.einsum("tgk,ngk->tng", xq.astype(np.int64).reshape(count, cols // G, G),
                    W.astype(np.int64).reshape(rows, cols // G, G))
    assert np.array_equal(acc.astype(np.int64), ref)


@pytest.mark.parametrize("form", [oracle.FORM_PANEL, oracle.FORM_PLANE])
def test_epilogue_against_float64(form):
    rng = np.random.default_rng(11 + form)
    W, sW = _matrix(rng, 512, 2048)
    x = rng.standard_normal((4, 2048)).astype(np.float32)
    y, acc, codes, scales = oracle.multiply(form, W, sW, x, with_acc=True)
    ref = np.einsum("tng,ng->tn", acc.astype(np.float64), sW.astype(np.float64)) * scales[:, None].astype(np.float64)
    scale = np.abs(ref).max()
    assert np.max(np.abs(y - ref)) < 1e-5 * scale
    # the codes are the per-row quantisation of ops.rs:112-118
    for t in range(4):
        c, s = oracle.quantise_int8(x[t])
        assert np.array_equal(codes[t], c) and scales[t] == s


def test_plane_epilogue_sequential_order():
    """neon.rs:180 evaluated in float32 left to right, group by group."""
    rng = np.random.default_rng(12)
    W, sW = _matrix(rng, 64, 512)
    xq = rng.integers(-128, 128, size=(1, 512), dtype=np.int8)
    sx = np.float32(0.0213)
    y, acc = oracle.product(oracle.FORM_PLANE, W, sW, xq, np.array([sx]), with_acc=True)
    for n in range(64):
        total = np.float32(0)
        for g in range(16):
            total = np.float32(total + np.float32(np.float32(acc[0, n, g]) * sW[n, g]) * sx)
        assert y[0, n] == total


def _round_f32(fr: Fraction) -> np.float32:
    """Correctly rounded (nearest, ties to even) float32 of an exact rational."""
    x = np.float32(float(fr))
    best = x
    for cand in (np.nextafter(x, np.float32(-np.inf)), np.nextafter(x, np.float32(np.inf))):
        d_best, d_cand = abs(Fraction(float(best)) - fr), abs(Fraction(float(cand)) - fr)
        if d_cand < d_best or (d_cand == d_best and (int(cand.view(np.uint32)) & 1) == 0):
            best = cand
    return np.float32(best)


def test_panel_epilogue_is_fused_multiply_add():
    """panel.rs:184-188: total = fma(acc, sW*sx, total) — one rounding per group.
    The fma is emulated with exact rationals; the input is chosen so that the
    unfused form (two roundings) differs on some rows, i.e. the check bites."""
    rng = np.random.default_rng(13)
    W, sW = _matrix(rng, 256, 512)
    xq = rng.integers(-128, 128, size=(1, 512), dtype=np.int8)
    sx = np.float32(0.0371)
    y, acc = oracle.product(oracle.FORM_PANEL, W, sW, xq, np.array([sx]), with_acc=True)
    differs = 0
    for n in range(256):
        fused = np.float32(0)
        unfused = np.float32(0)
        for g in range(16):
            s = np.float32(sW[n, g] * sx)
            fused = _round_f32(Fraction(int(acc[0, n, g])) * Fraction(float(s)) + Fraction(float(fused)))
            unfused = np.float32(unfused + np.float32(np.float32(acc[0, n, g]) * s))
        assert y[0, n] == fused, n
        differs += int(fused != unfused)
    assert differs > 0


# ---- attention -----------------------------------------------------------------------

def _attend64(q, K, V):
    s = (K.astype(np.float64) @ q.astype(np.float64)) / 8.0
    e = np.exp(s - s.max())
    return (e[:, None] * V.astype(np.float64)).sum(0) / e.sum()


@pytest.mark.parametrize("length", [1, 2, 15, 16, 17, 100, 544])
def test_attend_head_against_float64(length):
    rng = np.random.default_rng(length)
    q = rng.standard_normal(64).astype(np.float32) * 3
    K = rng.standard_normal((length, 64)).astype(np.float16)
    V = rng.standard_normal((length, 64)).astype(np.float16)
    out = oracle.attend_head(q, K, V)
    ref = _attend64(q, K, V)
    assert np.max(np.abs(out - ref)) < 2e-5 * max(1.0, np.abs(ref).max())


def test_attend_head_known_answers():
    rng = np.random.default_rng(21)
    V = rng.standard_normal((1, 64)).astype(np.float16)
    q = rng.standard_normal(64).astype(np.float32)
    K = rng.standard_normal((1, 64)).astype(np.float16)
    # one position: weight fast_exp(0) = 1, total 1, output = v exactly
    assert np.array_equal(oracle.attend_head(q, K, V), V[0].astype(np.float32))
    # identical keys: every weight is 1, output is the interleaved mean of the values
    K8 = np.repeat(K, 32, axis=0)
    V8 = rng.standard_normal((32, 64)).astype(np.float16)
    out = oracle.attend_head(q, K8, V8)
    assert np.allclose(out, V8.astype(np.float64).mean(0), atol=1e-6)
    # a dominant key picks its value
    Kd = np.zeros((40, 64), np.float16)
    Kd[23] = 50.0
    qd = np.ones(64, np.float32)
    assert np.allclose(oracle.attend_head(qd, Kd, V8.repeat(2, axis=0)[:40]), V8.repeat(2, axis=0)[23], atol=1e-6)

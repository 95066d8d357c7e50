"""The GPU quantiser multiplies by the reciprocal of the scale and falls back to
the division only near a rounding boundary (quantise_one_r in
rustyneedle_amd/csrc/rn_device.hpp). This restates that rule in IEEE float32
(numpy) and checks it against the defining division of ops.rs:112-118 on random
and adversarial inputs: quotients within a few ulps of every half-integer, for
scales over sixty decades."""
from __future__ import annotations

import numpy as np

f32 = np.float32


def reciprocal_rule(v: np.ndarray, s: np.float32) -> np.ndarray:
    r = f32(1) / s
    y = (v * r).astype(f32)
    h = (np.floor(y) + f32(0.5)).astype(f32)
    thr = (np.abs(y) * f32(2.0 ** -21) + f32(2.0 ** -30)).astype(f32)
    near = np.abs((y - h).astype(f32)) <= thr
    y = np.where(near, (v / s).astype(f32), y)
    return np.clip(np.rint(y), -128, 127)


def division_rule(v: np.ndarray, s: np.float32) -> np.ndarray:
    return np.clip(np.rint((v / s).astype(f32)), -128, 127)


def test_reciprocal_rule_equals_division():
    rng = np.random.default_rng(3)
    with np.errstate(over="ignore", invalid="ignore"):
        for _ in range(40):
            peak = f32(10.0 ** rng.uniform(-30, 30))
            s = f32(peak / f32(127))
            v = (rng.uniform(-1, 1, 50000) * peak).astype(f32)
            k = rng.integers(-128, 128, 50000).astype(f32)
            near = ((k + f32(0.5)) * s).astype(f32)
            steps = rng.integers(-4, 5, near.size)
            for u in range(1, 5):
                near = np.where(steps >= u, np.nextafter(near, f32(np.inf)), near)
                near = np.where(steps <= -u, np.nextafter(near, f32(-np.inf)), near)
            v = np.concatenate([v, near, np.array([peak, -peak, 0.0, -0.0, np.nan, np.inf], f32)])
            a, b = reciprocal_rule(v, s), division_rule(v, s)
            same = (a == b) | (np.isnan(a) & np.isnan(b))
            assert same.all(), (peak, v[~same][:4])

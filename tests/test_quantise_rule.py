"""The GPU quantiser's two division-free shortcuts (rustyneedle_amd/csrc/rn_device.hpp),
checked against the defining divisions of ops.rs:103-118 in IEEE float32:

- quotients: multiply by v_rcp_f32(scale), which is within 1 ulp of 1/scale, and
  fall back to the division near a rounding boundary (|fract(y) - 0.5| at most
  fma(|y|, 2^-21, 2^-30)) or for scales outside [2^-100, 2^100]. Restated in numpy for each of the three reciprocals a 1-ulp
  error allows, on random and adversarial inputs (quotients within a few ulps of
  every half-integer) for scales over sixty decades;
- int8_scale_from_peak: peak / 127 as q0 = peak * RN(1/127) plus one fma
  correction, compared with the division by a small C program (every 97th
  positive float here; all of them with RN_EXHAUSTIVE=1)."""
from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest

f32 = np.float32
HERE = os.path.dirname(os.path.abspath(__file__))


def reciprocal_rule(v: np.ndarray, s: np.float32, ulps: int = 0) -> np.ndarray:
    r = f32(1) / s
    for _ in range(abs(ulps)):
        r = np.nextafter(r, f32(np.inf) if ulps > 0 else f32(-np.inf))
    y = (v * r).astype(f32)
    # the device's test: d = v_fract_f32(y) - 0.5 (the fraction y - floor(y),
    # held below 1.0 as v_fract_f32 holds it), against fma(|y|, 2^-21, 2^-30),
    # one rounding (the float64 sum is exact: |y| * 2^-21 is a power-of-two
    # scaling); for |y| >= 2^23 the fraction is 0 and d = -0.5, never near
    frac = np.minimum((y - np.floor(y)).astype(f32), f32(np.nextafter(f32(1), f32(0))))
    d = (frac - f32(0.5)).astype(f32)
    thr = (np.abs(y).astype(np.float64) * 2.0 ** -21 + 2.0 ** -30).astype(f32)
    near = np.abs(d) <= thr
    if not (f32(2.0 ** -100) <= s <= f32(2.0 ** 100)):
        near = np.ones_like(near)
    # per element: the device sends a whole wave to the division when any lane
    # is near, which only replaces more quotients by the exact ones
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
            b = division_rule(v, s)
            for ulps in (-1, 0, 1):
                a = reciprocal_rule(v, s, ulps)
                same = (a == b) | (np.isnan(a) & np.isnan(b))
                assert same.all(), (peak, ulps, v[~same][:4])


def test_scale_without_division_matches_division(tmp_path):
    exe = tmp_path / "scale127"
    subprocess.run(["gcc", "-O2", "-march=x86-64-v3", "-ffp-contract=off", "-fopenmp",
                    os.path.join(HERE, "c", "scale127.c"), "-o", str(exe), "-lm"], check=True)
    stride = "1" if os.environ.get("RN_EXHAUSTIVE") else "97"
    out = subprocess.run([str(exe), stride], check=True, capture_output=True, text=True).stdout.split()
    bad, checked = int(out[0]), int(out[1])
    assert checked > 2_000_000 and bad == 0

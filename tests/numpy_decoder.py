"""An independent float64 NumPy model of the Needle-style decoder step.

Written from the reference's definitions, not from the oracle's code: it shares
no reduction order with the oracle (every sum is a float64 BLAS/NumPy sum), uses
libm-exact `exp` instead of `fast_exp`, float64 rotary angles and float64 norms.
What it does share is the model's definition, which is discrete and must match:
activations are quantised per row to int8 before each product
(crates/kernels/src/ops.rs:103-118: scale = absmax/127, 1 if all zero; round
half to even; clamp to [-128, 127]); the cache holds fp16 K/V; the embedding
row is dequantised and scaled by sqrt(d) (crates/model/src/session.rs:85-90);
the logits are the tied product of the quantised final hidden
(session.rs:166-177); greedy takes the first index of the maximum
(crates/generate/src/generator.rs:157-165).

Used by the tests as a second, independent check of the oracle's decoder.
"""
from __future__ import annotations

import numpy as np


def quantise(x: np.ndarray):
    peak = float(np.max(np.abs(x))) if x.size else 0.0
    scale = peak / 127.0 if peak > 0 else 1.0
    return np.clip(np.rint(x / scale), -128, 127), scale


def product(codes: np.ndarray, scales: np.ndarray, x: np.ndarray, group: int = 32) -> np.ndarray:
    """y = W_dequantised @ quantise(x), all in float64."""
    q, sx = quantise(x)
    rows, cols = codes.shape
    Wd = codes.astype(np.float64) * np.repeat(scales.astype(np.float64), group, axis=1)
    return (Wd @ q) * sx


def norm(x: np.ndarray, gain: np.ndarray, eps: float) -> np.ndarray:
    return x * (1.0 + gain.astype(np.float64)) / np.sqrt(np.mean(x * x) + eps)


def rotary(head: np.ndarray, pos: int, theta: float) -> np.ndarray:
    half = head.size // 2
    i = np.arange(half, dtype=np.float64)
    angle = pos * theta ** (-2.0 * i / head.size)
    c, s = np.cos(angle), np.sin(angle)
    a, b = head[:half], head[half:]
    return np.concatenate([a * c - b * s, b * c + a * s])


def silu(x: np.ndarray) -> np.ndarray:
    return x / (1.0 + np.exp(-x))


class Decoder:
    """cfg: the model configuration dict; weights: the dict of host tensors
    (codes int8, scales f32, gains f32) keyed like rustyneedle_amd.synthetic_weights."""

    def __init__(self, cfg: dict, weights: dict, capacity: int):
        self.c, self.w = cfg, weights
        L, H, hd = cfg["layers"], cfg["heads"], cfg["head_dim"]
        self.K = np.zeros((L, H, capacity, hd), dtype=np.float16)
        self.V = np.zeros((L, H, capacity, hd), dtype=np.float16)
        self.length = 0

    def set_cache(self, keys: np.ndarray, values: np.ndarray) -> None:
        n = keys.shape[2]
        self.K[:, :, :n] = keys.view(np.float16)
        self.V[:, :, :n] = values.view(np.float16)
        self.length = n

    def push(self, token: int) -> np.ndarray:
        """One step; returns the float64 logits."""
        c, w = self.c, self.w
        d, H, hd, f = c["d_model"], c["heads"], c["head_dim"], c["ffn"]
        eps, theta = c["norm_eps"], c["rope_theta"]
        pos = self.length
        ec, es = w["embedding"]
        x = ec[token].astype(np.float64) * np.repeat(es[token].astype(np.float64), 32) * np.sqrt(d)
        for l, lw in enumerate(w["layers"]):
            qkv = product(*lw["qkv"], norm(x, lw["norm_attn"], eps))
            q, k, v = qkv[:d], qkv[d:2 * d], qkv[2 * d:]
            att = np.empty(d)
            for h in range(H):
                sl = slice(h * hd, (h + 1) * hd)
                self.K[l, h, pos] = rotary(k[sl], pos, theta).astype(np.float16)
                self.V[l, h, pos] = v[sl].astype(np.float16)
                Kh = self.K[l, h, :pos + 1].astype(np.float64)
                Vh = self.V[l, h, :pos + 1].astype(np.float64)
                s = Kh @ rotary(q[sl], pos, theta) / np.sqrt(hd)
                p = np.exp(s - s.max())
                att[sl] = (p / p.sum()) @ Vh
            x = x + product(*lw["out"], att)
            gu = product(*lw["gate_up"], norm(x, lw["norm_ffn"], eps))
            x = x + product(*lw["down"], silu(gu[:f]) * gu[f:])
        self.length = pos + 1
        hidden = norm(x, w["norm_final"], eps)
        return product(*w["embedding"], hidden)

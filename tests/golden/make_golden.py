"""Writes the golden fixtures of this directory from the oracle.

Fixtures (numpy .npz, no pickles):

- gemv_2048x512.npz — the single int8 matvec: x f32[512] ~ N(0,1); codes
  U{-127..127} [2048][512] and scales U[1e-3,1e-2] [2048][16] drawn by the
  seeded generator under the names "gemv.codes" / "gemv.scales" (SHA-256 of
  their bytes stored so a drifting generator is caught); outputs: the
  per-row activation codes and scale, acc int32 [2048][16], y f32 [2048]
  (panel epilogue).
- decode_20l_16.npz — the 20-layer d=512 decoder with the seeded synthetic
  weights, fp16 cache of 256 N(0,1) positions ("decode.k"/"decode.v"), first
  token "decode.first": 16 greedy ids and the logits of the first step.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
import rustyneedle_amd as rn  # noqa: E402

CONTEXT = 256
STEPS = 16


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def gemv_inputs():
    W = rn.synth_codes(rn.SEED, "gemv.codes", (2048, 512))
    sW = rn.synth_uniform(rn.SEED, "gemv.scales", 1e-3, 1e-2, (2048, 16))
    x = rn.synth_normal(rn.SEED, "gemv.x", 1.0, (512,))
    return W, sW, x


def decode_inputs():
    cfg = dict(rn.NEEDLE_DECODER)
    weights = rn.synthetic_weights(cfg)
    keys, values = rn.synthetic_cache(cfg, CONTEXT, "decode")
    first = int(rn.synth_tokens(rn.SEED, "decode.first", cfg["vocab"], 1)[0])
    return cfg, weights, keys, values, first


def main() -> None:
    W, sW, x = gemv_inputs()
    y, acc, codes, scales = oracle.multiply(oracle.FORM_PANEL, W, sW, x, with_acc=True)
    np.savez_compressed(os.path.join(HERE, "gemv_2048x512.npz"), x=x, xq=codes[0], sx=scales,
                        acc=acc[0], y=y[0], codes_sha256=np.array(sha(W)), scales_sha256=np.array(sha(sW)))

    cfg, weights, keys, values, first = decode_inputs()
    om = oracle.OracleModel(cfg, weights)
    s = om.session(CONTEXT + STEPS)
    s.set_cache(keys, values)
    s.push(first)
    logits0 = s.logits()
    s = om.session(CONTEXT + STEPS)
    s.set_cache(keys, values)
    ids = s.greedy(first, STEPS)
    np.savez_compressed(os.path.join(HERE, "decode_20l_16.npz"), first=np.array(first, dtype=np.uint32),
                        ids=ids, logits0=logits0, context=np.array(CONTEXT),
                        embedding_sha256=np.array(sha(weights["embedding"][0])),
                        keys_sha256=np.array(sha(keys)))
    print("first", first, "ids", ids.tolist())


if __name__ == "__main__":
    main()

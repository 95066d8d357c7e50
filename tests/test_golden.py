"""The oracle against the committed golden fixtures, closed forms and an
independent float64 model of the decoder (no GPU)."""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_golden  # noqa: E402
import numpy_decoder  # noqa: E402
import oracle  # noqa: E402
import rustyneedle_amd as rn  # noqa: E402

GOLDEN = os.path.join(HERE, "golden")


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def gemv():
    return np.load(os.path.join(GOLDEN, "gemv_2048x512.npz"), allow_pickle=False)


@pytest.fixture(scope="module")
def decode():
    return np.load(os.path.join(GOLDEN, "decode_20l_16.npz"), allow_pickle=False)


@pytest.fixture(scope="module")
def decode_inputs():
    return make_golden.decode_inputs()


def test_gemv_inputs_regenerate(gemv):
    W, sW, x = make_golden.gemv_inputs()
    assert sha(W) == str(gemv["codes_sha256"])
    assert sha(sW) == str(gemv["scales_sha256"])
    assert np.array_equal(x.view(np.uint32), gemv["x"].view(np.uint32))


def test_gemv_oracle_matches_fixture(gemv):
    W, sW, x = make_golden.gemv_inputs()
    y, acc, codes, scales = oracle.multiply(oracle.FORM_PANEL, W, sW, x, with_acc=True)
    assert np.array_equal(codes[0], gemv["xq"])
    assert np.array_equal(scales.view(np.uint32), gemv["sx"].view(np.uint32))
    assert np.array_equal(acc[0], gemv["acc"])
    assert np.array_equal(y[0].view(np.uint32), gemv["y"].view(np.uint32))


def test_gemv_fixture_closed_form(gemv):
    """Independent of the oracle: codes = rint(x / (absmax/127)) clamped, acc the
    exact integer group sums, y the float64 epilogue within float32 rounding."""
    W, sW, x = make_golden.gemv_inputs()
    sx = np.float32(np.max(np.abs(x))) / np.float32(127.0)
    assert np.float32(gemv["sx"][0]) == sx
    xq = np.clip(np.rint(x / sx), -128, 127).astype(np.int8)
    assert np.array_equal(xq, gemv["xq"])
    acc = np.einsum("rgk,gk->rg", W.reshape(2048, 16, 32).astype(np.int64), xq.reshape(16, 32).astype(np.int64))
    assert np.array_equal(acc, gemv["acc"].astype(np.int64))
    y64 = (acc.astype(np.float64) * sW.astype(np.float64)).sum(axis=1) * float(sx)
    assert np.allclose(gemv["y"].astype(np.float64), y64, rtol=1e-5, atol=1e-6 * np.max(np.abs(y64)))


def test_decode_oracle_matches_fixture(decode, decode_inputs):
    cfg, weights, keys, values, first = decode_inputs
    assert int(decode["first"]) == first
    assert sha(weights["embedding"][0]) == str(decode["embedding_sha256"])
    assert sha(keys) == str(decode["keys_sha256"])
    om = oracle.OracleModel(cfg, weights)
    s = om.session(make_golden.CONTEXT + make_golden.STEPS)
    s.set_cache(keys, values)
    ids = s.greedy(first, make_golden.STEPS)
    assert ids.tolist() == decode["ids"].tolist()
    s = om.session(make_golden.CONTEXT + 1)
    s.set_cache(keys, values)
    s.push(first)
    assert np.array_equal(s.logits().view(np.uint32), decode["logits0"].view(np.uint32))


def test_float64_model_one_and_two_layers():
    """Every op of the decoder step (embedding, norms, fused QKV, rotary, fp16
    append, attention, out, gated FFN, final norm, tied logits) against the
    float64 model. Per-row int8 quantisation makes the model discontinuous: a
    value within float32 rounding of a rounding boundary flips one code and
    moves the logits by ~1e-3, so most cases must agree to float32 rounding
    and none may differ by more than such a flip."""
    rel = []
    for layers in (1, 2):
        cfg = dict(rn.NEEDLE_DECODER)
        cfg.update(layers=layers, vocab=1000)
        w = rn.synthetic_weights(cfg, seed=5)
        om = oracle.OracleModel(cfg, w)
        for ctx in (0, 3, 40):
            keys, values = rn.synthetic_cache(cfg, max(ctx, 1), f"f64.{ctx}", seed=5)
            dec = numpy_decoder.Decoder(cfg, w, ctx + 8)
            s = om.session(ctx + 8)
            if ctx:
                dec.set_cache(keys[:, :, :ctx], values[:, :, :ctx])
                s.set_cache(keys[:, :, :ctx], values[:, :, :ctx])
            for tok in (1, 500, 999):
                l64 = dec.push(tok)
                s.push(tok)
                l32 = s.logits().astype(np.float64)
                rel.append(np.linalg.norm(l64 - l32) / np.linalg.norm(l64))
    rel = np.array(rel)
    assert np.all(rel < 1e-2), rel
    assert np.mean(rel < 1e-6) >= 0.8, rel


def test_float64_model_full_decoder(decode, decode_inputs):
    """The 20-layer fixture decode, teacher-forced through the float64 model:
    with ~0.4 code flips per token the random-init model drifts by a few
    percent, so this bounds gross errors (a wrong layer, head or operand
    gives relative differences of order 1)."""
    cfg, weights, keys, values, first = decode_inputs
    dec = numpy_decoder.Decoder(cfg, weights, make_golden.CONTEXT + 4)
    dec.set_cache(keys, values)
    om = oracle.OracleModel(cfg, weights)
    s = om.session(make_golden.CONTEXT + 4)
    s.set_cache(keys, values)
    tok = first
    for step in range(3):
        l64 = dec.push(tok)
        s.push(tok)
        l32 = s.logits().astype(np.float64)
        rel = np.linalg.norm(l64 - l32) / np.linalg.norm(l64)
        assert rel < 0.2, (step, rel)
        assert np.corrcoef(l64, l32)[0, 1] > 0.98
        tok = int(decode["ids"][step])

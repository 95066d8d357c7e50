"""The Whistle-style oracle (oracle/rn_whistle.c) against an independent float64
model (tests/numpy_whistle.py) and known answers (no GPU)."""
from __future__ import annotations

import numpy as np
import pytest

import numpy_whistle as nw
import oracle
import rustyneedle_amd as rn


@pytest.fixture(scope="module")
def small():
    cfg = dict(rn.WHISTLE)
    cfg.update(frames=64, enc_layers=1, dec_layers=1, vocab=1000)
    w = rn.synthetic_whistle_weights(cfg, seed=3)
    return cfg, w, oracle.OracleWhistle(cfg, w), rn.synthetic_mel(cfg, seed=3)


def row_rel(a, b):
    a, b = np.atleast_2d(a).astype(np.float64), np.atleast_2d(b).astype(np.float64)
    return np.linalg.norm(a - b, axis=1) / np.maximum(np.linalg.norm(b, axis=1), 1e-30)


def test_sigmoid_and_position_table():
    assert oracle.sigmoid(0.0) == 0.5
    gate = oracle.sigmoid(0.3)
    tab = oracle.whistle_position_table(50, 384, gate)
    ref = nw.position_table(50, 384, gate)
    assert np.max(np.abs(tab - ref)) < 2e-5  # angles up to 49 rad in float32
    assert np.all(tab[0, :192] == 0.0) and np.allclose(tab[0, 192:], gate)


def test_int8_attend_against_float64_and_known_answers():
    rng = np.random.default_rng(0)
    qc = rng.integers(-127, 128, 64).astype(np.int8)
    kc = rng.integers(-127, 128, (300, 64)).astype(np.int8)
    vc = rng.integers(-127, 128, (300, 64)).astype(np.int8)
    ks = rng.uniform(1e-3, 1e-2, 300).astype(np.float32)
    vs = rng.uniform(1e-3, 1e-2, 300).astype(np.float32)
    a = oracle.int8_attend(qc, 0.01, kc, ks, vc, vs)
    b = nw.int8_attend(qc, 0.01, kc, ks.astype(np.float64), vc, vs.astype(np.float64))
    assert np.max(np.abs(a - b)) <= 3e-6 * np.max(np.abs(b))
    # identical keys: the weights are uniform, the output the mean of scaled values
    same = np.repeat(kc[:1], 40, axis=0)
    out = oracle.int8_attend(qc, 0.01, same, np.full(40, ks[0]), vc[:40], np.ones(40, np.float32))
    assert np.allclose(out, vc[:40].astype(np.float64).mean(axis=0), rtol=1e-5, atol=1e-5)
    # one dominant key: its value row comes out
    k2 = kc[:10].copy()
    k2[3] = qc
    out = oracle.int8_attend(qc, 1.0, k2, np.ones(10, np.float32), vc[:10], np.ones(10, np.float32))
    assert np.array_equal(out, vc[3].astype(np.float32))


def test_stem_against_float64(small):
    cfg, w, o, mel = small
    st, ref = o.stem(mel), nw.stem(cfg, w, mel)
    assert st.shape == (32, 384)
    rel = row_rel(st, ref)
    # a second-convolution input code within float32 rounding of a rounding boundary may
    # flip (the model is discontinuous there); every other row agrees to float32
    assert np.mean(rel < 1e-5) >= 0.9, rel
    assert np.all(rel < 2e-2), rel


def test_encoder_layer_against_float64(small):
    cfg, w, o, mel = small
    x = o.stem(mel)
    rel = row_rel(o.encoder_layer(0, x), nw.encoder_layer(cfg, w["enc"][0], x.astype(np.float64)))
    assert np.mean(rel < 1e-5) >= 0.9, rel
    assert np.all(rel < 2e-2), rel


def test_memory_and_decoder_against_float64(small):
    cfg, w, o, mel = small
    enc = o.encode(mel)
    mk, ks, mv, vs = o.memory(enc)
    ref = nw.memory(cfg, w, enc.astype(np.float64))
    assert np.mean(mk[0] == ref[0][0]) > 0.999 and np.mean(mv[0] == ref[0][2]) > 0.999
    assert np.allclose(ks[0], ref[0][1], rtol=1e-6) and np.allclose(vs[0], ref[0][3], rtol=1e-6)
    s = o.session(8, (mk, ks, mv, vs))
    dec = nw.Decoder(cfg, w, ref, 8)
    rel = []
    for tok in (5, 17, 999, 0):
        s.push(tok)
        rel.append(row_rel(s.logits(), dec.push(tok))[0])
    rel = np.array(rel)
    assert np.mean(rel < 1e-5) >= 0.75 and np.all(rel < 2e-2), rel


def test_greedy_equals_push_and_argmax(small):
    cfg, w, o, mel = small
    mem = o.memory(o.encode(mel))
    ids = o.session(8, mem).greedy(7, 5)
    s = o.session(8, mem)
    tok, got = 7, []
    for _ in range(5):
        s.push(tok)
        tok = oracle.argmax(s.logits())
        got.append(tok)
    assert ids.tolist() == got

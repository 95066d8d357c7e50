"""The speech path on the GPU against the oracle, bit for bit, through the C ABI."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import rustyneedle_amd as rn

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.fixture(scope="module")
def small():
    cfg = dict(rn.WHISTLE)
    cfg.update(frames=64, enc_layers=2, dec_layers=2, vocab=1000, max_positions=24)
    w = rn.synthetic_whistle_weights(cfg, seed=11)
    return cfg, oracle.OracleWhistle(cfg, w), rn.Whistle(cfg, seed=11), rn.synthetic_mel(cfg, seed=11)


def test_host_tables(small):
    cfg, o, g, _ = small
    pos, gains = g.tables()
    assert np.array_equal(_bits(pos), _bits(o.position))
    ref = np.array([oracle.sigmoid(lw["gate"]) for lw in o.w["dec"]], np.float32)
    assert np.array_equal(_bits(gains), _bits(ref))


def test_stem(small):
    cfg, o, g, mel = small
    assert np.array_equal(_bits(g.stem(mel)), _bits(o.stem(mel)))


def test_encode_and_memory(small):
    cfg, o, g, mel = small
    enc = g.encode(mel)
    ref = o.encode(mel)
    assert np.array_equal(_bits(enc), _bits(ref))
    for a, b in zip(g.memory(), o.memory(ref)):
        assert np.array_equal(a.view(np.uint8) if a.dtype == np.int8 else _bits(a),
                              b.view(np.uint8) if b.dtype == np.int8 else _bits(b))


def test_push_logits_and_greedy(small):
    cfg, o, g, mel = small
    enc = g.encode(mel)
    mem = o.memory(o.encode(mel))
    s = o.session(cfg["max_positions"], mem)
    for tok in (3, 999, 0):
        g.push(tok)
        s.push(tok)
        assert np.array_equal(_bits(g.logits()), _bits(s.logits()))
    g.reset()
    ids = g.decode_greedy(7, 12)
    assert ids.tolist() == o.session(cfg["max_positions"], mem).greedy(7, 12).tolist()
    with pytest.raises(rn.RnError):
        g.decode_greedy(7, 13)  # 12 + 13 positions exceed the 24 of the session
    assert enc.shape == (32, 384)


def test_full_size_encode_and_48_tokens():
    """The 3000-frame, 6-encoder-layer, 4-decoder-layer configuration."""
    cfg = dict(rn.WHISTLE)
    w = rn.synthetic_whistle_weights(cfg)
    o = oracle.OracleWhistle(cfg, w)
    g = rn.Whistle(cfg)
    mel = rn.synthetic_mel(cfg)
    oracle.set_threads(8)
    enc = g.encode(mel)
    ref = o.encode(mel)
    assert np.array_equal(_bits(enc), _bits(ref))
    first = int(rn.synth_tokens(rn.SEED, "whistle.first", cfg["vocab"], 1)[0])
    ids = g.decode_greedy(first, 48)
    assert ids.tolist() == o.session(cfg["max_positions"], o.memory(ref)).greedy(first, 48).tolist()


def test_d512_eight_heads():
    """d_model 512 (8 heads, FFN 2048): the 512-wide cross kernel, class-sum and
    cross-norm prologues and the 8-head encoder attention, against the oracle."""
    cfg = dict(rn.WHISTLE)
    cfg.update(d_model=512, heads=8, ffn=2048, frames=80, enc_layers=1, dec_layers=2, vocab=1000, max_positions=16)
    w = rn.synthetic_whistle_weights(cfg, seed=13)
    o, g, mel = oracle.OracleWhistle(cfg, w), rn.Whistle(cfg, seed=13), rn.synthetic_mel(cfg, seed=13)
    enc = g.encode(mel)
    ref = o.encode(mel)
    assert enc.shape == (40, 512)
    assert np.array_equal(_bits(enc), _bits(ref))
    mem = o.memory(ref)
    s = o.session(cfg["max_positions"], mem)
    for tok in (2, 999, 31):
        g.push(tok)
        s.push(tok)
        assert np.array_equal(_bits(g.logits()), _bits(s.logits()))
    g.reset()
    assert g.decode_greedy(5, 10).tolist() == o.session(cfg["max_positions"], mem).greedy(5, 10).tolist()


@pytest.mark.parametrize("mel_frames", [2, 17, 100])
def test_ragged_frame_counts(mel_frames):
    """1, 9 and 50 encoder frames: a single frame, a last query tile of one, a
    head's values shorter than one staging pass."""
    cfg = dict(rn.WHISTLE)
    cfg.update(frames=mel_frames, enc_layers=1, dec_layers=1, vocab=500, max_positions=8)
    w = rn.synthetic_whistle_weights(cfg, seed=5)
    o, g, mel = oracle.OracleWhistle(cfg, w), rn.Whistle(cfg, seed=5), rn.synthetic_mel(cfg, seed=5)
    enc = g.encode(mel)
    ref = o.encode(mel)
    assert enc.shape == ((mel_frames - 1) // 2 + 1, 384)
    assert np.array_equal(_bits(enc), _bits(ref))
    s = o.session(cfg["max_positions"], o.memory(ref))
    for tok in (4, 499):
        g.push(tok)
        s.push(tok)
        assert np.array_equal(_bits(g.logits()), _bits(s.logits()))


def test_host_weights_equal_synthetic_and_oracle():
    """rn_whistle_create over host weights (Whistle::open's role, lib.rs:101-140)
    builds the same model as the library's seeded draws: stem, encode and greedy
    ids equal, and equal to the oracle; weights perturbed on the host change the
    result (the host arrays are the ones used)."""
    cfg = dict(rn.WHISTLE)
    cfg.update(frames=40, enc_layers=1, dec_layers=1, vocab=500, max_positions=16)
    w = rn.synthetic_whistle_weights(cfg, seed=5)
    a, b = rn.Whistle(cfg, seed=5), rn.Whistle(cfg, weights=w)
    mel = rn.synthetic_mel(cfg, seed=5)
    o = oracle.OracleWhistle(cfg, w)
    assert np.array_equal(_bits(a.stem(mel)), _bits(b.stem(mel)))
    enc = b.encode(mel)
    assert np.array_equal(_bits(a.encode(mel)), _bits(enc))
    assert np.array_equal(_bits(enc), _bits(o.encode(mel)))
    ids = b.decode_greedy(3, 6)
    assert ids.tolist() == a.decode_greedy(3, 6).tolist()
    assert ids.tolist() == o.session(cfg["max_positions"], o.memory(o.encode(mel))).greedy(3, 6).tolist()
    w2 = dict(w)
    w2["conv2"] = (w["conv2"][0].copy(), w["conv2"][1] * np.float32(2.0))
    c = rn.Whistle(cfg, weights=w2)
    assert not np.array_equal(_bits(c.stem(mel)), _bits(b.stem(mel)))

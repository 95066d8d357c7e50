"""The Needle 3 token step on the GPU (crates/model/src/session.rs) against the
oracle, bit for bit, on a synthetic archive with every feature of the block:
four lanes, two engram sites (layers 0 and 2; orders 2 and 3, dilation 2),
conv taps on q/k/v, grouped queries (4 heads over 2 kv heads), a 16-token
window with layer 1 global, the Hadamard MLP, two probe heads (a 3-bit head
projection on the float path), 4-bit embedding and tables, 2-bit projections.

Each push compares the hidden state and every cell; at the end the logits,
both heads' pooled readouts and outputs, and every layer's int8 cache (codes
and scales). 40 tokens run past the window. A depth-2 ladder model (layers 0
and 3) leaves the engram site of layer 2 out."""
import numpy as np
import pytest

import oracle
import rustyneedle_amd as rn
from rustyneedle_amd import needle3

pytestmark = pytest.mark.gpu

GEOMETRY = needle3.NEEDLE3_SMALL


@pytest.fixture(scope="module")
def archive():
    return needle3.synthetic_archive(GEOMETRY)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _tokens(n, seed=3):
    return rn.synth_tokens(seed, "needle3.tokens", GEOMETRY["vocab"], (n,))


def _compare_session(gs, os_, label):
    assert np.array_equal(_bits(gs.logits()), _bits(os_.logits())), label
    for code in (1, 2):
        assert np.array_equal(_bits(gs.pooled_readout(code)), _bits(os_.pooled_readout(code))), (label, code)
        assert np.array_equal(_bits(gs.head_output(code)), _bits(os_.head_output(code))), (label, code)
    assert gs.head_output(3) is None and os_.head_output(3) is None


@pytest.fixture(params=["fused", "stepwise"])
def path(request, monkeypatch):
    """The three-kernel step and the one-launch-a-piece step (RN_N3_PATH)."""
    if request.param == "stepwise":
        monkeypatch.setenv("RN_N3_PATH", "stepwise")
    else:
        monkeypatch.delenv("RN_N3_PATH", raising=False)
    return request.param


@pytest.mark.parametrize("depth", [0, 2])
def test_push_bit_exact(archive, depth, path):
    gm = needle3.Model(archive, depth)
    om = oracle.OracleNeedle3(archive, depth)
    assert gm.active == om.active
    gs, os_ = gm.session(64), om.session(64)
    tokens = _tokens(40)
    for i, t in enumerate(tokens):
        print(f"needle3 {path} depth {depth} push {i}", flush=True)
        gs.push(int(t))
        os_.push(int(t))
        assert np.array_equal(_bits(gs.hidden()), _bits(os_.hidden())), f"hidden at step {i}"
        assert np.array_equal(_bits(gs.cells()), _bits(os_.cells())), f"cells at step {i}"
    assert len(gs) == len(os_) == 40
    _compare_session(gs, os_, f"depth {depth}")
    for layer in gm.active:
        g, o = gs.cache(layer), os_.cache(layer)
        for a, b in zip(g, o):
            assert a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8)), layer


def test_feed_equals_push(archive, path):
    gm = needle3.Model(archive)
    a, b = gm.session(64), gm.session(64)
    tokens = _tokens(21, seed=5)
    a.feed(tokens)
    for t in tokens:
        b.push(int(t))
    assert np.array_equal(_bits(a.logits()), _bits(b.logits()))
    assert np.array_equal(_bits(a.cells()), _bits(b.cells()))


def test_decode_greedy(archive, path):
    """Generator::run_turn's loop with the argmax on the device: the ids, then
    the state after them, against the oracle."""
    gm, om = needle3.Model(archive), oracle.OracleNeedle3(archive)
    gs, os_ = gm.session(64), om.session(64)
    prompt = _tokens(9, seed=11)
    gs.feed(prompt)
    os_.feed(prompt)
    ids = gs.decode_greedy(7, 24)
    want = os_.greedy(7, 24)
    assert ids.tolist() == want.tolist()
    assert len(gs) == len(os_) == 9 + 24
    assert np.array_equal(_bits(gs.hidden()), _bits(os_.hidden()))
    assert np.array_equal(_bits(gs.logits()), _bits(os_.logits()))


def test_errors(archive):
    gm = needle3.Model(archive)
    s = gm.session(4)
    with pytest.raises(rn.RnError):
        s.push(GEOMETRY["vocab"])
    s.feed([1, 2, 3, 4])
    with pytest.raises(rn.RnError):
        s.push(5)
    with pytest.raises(rn.RnError):
        needle3.Model(archive, depth=1)


def _compare_all(gs, os_, gm, label):
    assert len(gs) == len(os_), label
    assert np.array_equal(_bits(gs.hidden()), _bits(os_.hidden())), f"hidden {label}"
    assert np.array_equal(_bits(gs.cells()), _bits(os_.cells())), f"cells {label}"
    _compare_session(gs, os_, label)
    for layer in gm.active:
        for a, b in zip(gs.cache(layer), os_.cache(layer)):
            assert a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8)), (label, layer)


@pytest.mark.parametrize("chunk", [4, 7, 256])
@pytest.mark.parametrize("depth", [0, 2])
def test_batched_feed_bit_exact(archive, depth, chunk, monkeypatch):
    """Session::feed's batched prefill (prefill.rs:10-99): runs of up to
    `chunk` tokens (a last run under four tokens pushed), against the oracle
    pushing the same tokens, after each of three feeds (21 tokens, 3 tokens,
    which are pushed, then 30, past the 16-token window); with chunks of 4 and
    7 the conv-tap and engram rings (3 and 5 positions) cross run boundaries."""
    monkeypatch.delenv("RN_N3_PATH", raising=False)
    monkeypatch.setenv("RN_N3_FEED_CHUNK", str(chunk))
    gm, om = needle3.Model(archive, depth), oracle.OracleNeedle3(archive, depth)
    gs, os_ = gm.session(64), om.session(64)
    tokens = _tokens(54, seed=17)
    for a, b in ((0, 21), (21, 24), (24, 54)):
        print(f"needle3 batched feed depth {depth} chunk {chunk} tokens {a}..{b}", flush=True)
        gs.feed(tokens[a:b])
        os_.feed(tokens[a:b])
        _compare_all(gs, os_, gm, f"depth {depth} chunk {chunk} after {b}")
    # the session goes on by pushes and greedy decoding from the fed state
    ids = gs.decode_greedy(5, 6)
    assert ids.tolist() == os_.greedy(5, 6).tolist()
    _compare_all(gs, os_, gm, f"depth {depth} chunk {chunk} after greedy")

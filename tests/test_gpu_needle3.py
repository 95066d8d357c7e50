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
    # a layer the ladder leaves out has no cache (the reference never fills it)
    for layer in set(range(GEOMETRY["num_layers"])) - set(gm.active):
        with pytest.raises(rn.RnError):
            gs.cache(layer)


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


def test_clone_diverges_independently(archive, path):
    """#[derive(Clone)] on Session (session.rs:17), the Generator's prefix
    cache (generator.rs:41-46): after a batched feed the session is cloned;
    base and clone then take different tokens, and each matches an oracle
    session that took the same ones (state, heads, caches); a clone of the
    clone then feeds again while the clone stays as it was."""
    gm, om = needle3.Model(archive), oracle.OracleNeedle3(archive)
    gs, os_ = gm.session(96), om.session(96)
    prompt = _tokens(20, seed=23)
    gs.feed(prompt)
    os_.feed(prompt)
    gc, oc = gs.clone(), os_.clone()
    _compare_all(gc, oc, gm, "fresh clone")
    for t in _tokens(6, seed=29):
        gs.push(int(t))
        os_.push(int(t))
    for t in _tokens(9, seed=31):
        gc.push(int(t))
        oc.push(int(t))
    _compare_all(gs, os_, gm, "base after its tokens")
    _compare_all(gc, oc, gm, "clone after its tokens")
    gc2, oc2 = gc.clone(), oc.clone()
    more = _tokens(12, seed=37)
    gc2.feed(more)
    oc2.feed(more)
    _compare_all(gc2, oc2, gm, "clone of the clone after a feed")
    _compare_all(gc, oc, gm, "clone left as it was")
    assert gc2.decode_greedy(3, 5).tolist() == oc2.greedy(3, 5).tolist()


def test_run_turn_stops_like_the_generator(archive, path):
    """Generator::run_turn's loop (generator.rs:99-130): a turn without a stop
    token runs max_tokens; with a stop token planted from that turn's ids a
    turn from the same prefix (a clone) ends after pushing its first
    occurrence; a short window ends the loop at len + 1 == window. Ids,
    length, finished and the whole state (head_output(2) included, which the
    reference reads after the loop) against the oracle."""
    gm, om = needle3.Model(archive), oracle.OracleNeedle3(archive)
    gs, os_ = gm.session(96), om.session(96)
    prompt = _tokens(10, seed=41)
    gs.feed(prompt)
    os_.feed(prompt)
    base_g, base_o = gs.clone(), os_.clone()
    want, fin = os_.run_turn(20, 4096, [])
    got, gfin = gs.run_turn(20, window=4096)
    assert got.tolist() == want.tolist() and not fin and not gfin and len(want) == 20
    _compare_all(gs, os_, gm, "turn of 20")
    for k in (0, 7):
        stop = int(want[k])
        g2, o2 = base_g.clone(), base_o.clone()
        want2, fin2 = o2.run_turn(20, 4096, [GEOMETRY["vocab"] - 1, stop])
        got2, gfin2 = g2.run_turn(20, stops=[GEOMETRY["vocab"] - 1, stop], window=4096)
        assert fin2 and gfin2 and got2.tolist() == want2.tolist(), (k, got2, want2)
        stops_at = [i for i, t in enumerate(want.tolist()) if t in (stop, GEOMETRY["vocab"] - 1)]
        assert len(got2) == stops_at[0] + 1
        _compare_all(g2, o2, gm, f"stopped turn {k}")
        assert np.array_equal(_bits(g2.head_output(2)), _bits(o2.head_output(2)))
    g3, o3 = base_g.clone(), base_o.clone()
    want3, fin3 = o3.run_turn(50, len(o3) + 6, [])
    got3, gfin3 = g3.run_turn(50, window=len(g3) + 6)
    assert len(want3) == 5 and got3.tolist() == want3.tolist() and not gfin3
    _compare_all(g3, o3, gm, "window")
    with pytest.raises(rn.RnError):
        g3.run_turn(200, window=4096)  # 200 more tokens cannot fit the capacity of 96


def test_choose_allowed_on_the_session(archive):
    """generator.rs:104-116 on the Needle 3 session's logits: argmax_allowed
    with the argmax fallback and allowed_statistics, bit for bit; the chosen
    token is pushed and the next choice compared again."""
    gm, om = needle3.Model(archive), oracle.OracleNeedle3(archive)
    gs, os_ = gm.session(64), om.session(64)
    prompt = _tokens(12, seed=43)
    gs.feed(prompt)
    os_.feed(prompt)
    rng = np.random.default_rng(5)
    n = gm.output_vocab
    for mask in ((rng.random(n) < 0.3).astype(np.uint8), np.zeros(n, np.uint8), np.ones(n, np.uint8),
                 (rng.random(n) < 0.01).astype(np.uint8)):
        got = gs.choose_allowed(mask)
        want = os_.choose_allowed(mask)
        assert got[0] == want[0] and got[1] == bool(want[1]), (got, want)
        assert np.array_equal(_bits([got[2], got[3]]), _bits([want[2], want[3]]))
        gs.push(got[0])
        os_.push(want[0])
    _compare_all(gs, os_, gm, "after constrained steps")


@pytest.mark.parametrize("path", ["fused"], indirect=True)
def test_float_path_projections_feed_as_the_reference_prefills(path):
    """3-bit projections and engram matrices take the float path, whose batch
    tile (multiply_batch, matrix.rs:356-378) rounds differently from a push's
    vector product (test_needle3_oracle.py shows the oracle's feed and pushes
    differ there). Feeds of 21 tokens (a prefill), 2 (pushes) and 130 (a
    prefill of 128, then 2 pushes: the reference's PREFILL_CHUNK,
    session.rs:11, 56-70) run the batched path with the batch arithmetic and
    match the oracle's prefill-faithful feed bit for bit after each; then
    pushes and greedy tokens from the fed state."""
    bits = dict(needle3.BITS, projection=3, engram=3)
    archive = needle3.synthetic_archive(GEOMETRY, bits=bits)
    gm, om = needle3.Model(archive), oracle.OracleNeedle3(archive)
    gs, os_ = gm.session(200), om.session(200)
    tokens = _tokens(153, seed=47)
    for a, b in ((0, 21), (21, 23), (23, 153)):
        print(f"needle3 3-bit projections: feed of tokens {a}..{b}", flush=True)
        gs.feed(tokens[a:b])
        os_.feed(tokens[a:b])
        _compare_all(gs, os_, gm, f"3-bit after {b}")
    for t in (5, 77):
        gs.push(t)
        os_.push(t)
    assert gs.decode_greedy(9, 4).tolist() == os_.greedy(9, 4).tolist()
    _compare_all(gs, os_, gm, "3-bit after pushes and greedy tokens")

"""Pins of the Needle 3 oracle (oracle/rn_needle3.c), CPU only.

- The whole step against an independent float64 model (tests/numpy_needle3.py,
  written from the reference's Rust with NumPy and scipy's Hadamard matrix): the
  hidden state, every cell and the logits after each of 24 pushes past a
  16-token window, by cosine and relative error; the argmax of the logits. A
  dropped term (engram, conv taps, a norm, rotary, the gate, a lane) moves
  these by far more than the arithmetic the model leaves out.
- The Hadamard MLP: with identity factors and permutations, unit diagonals, a
  zero bias and zero condition rows it is silu of the input, exactly; against
  float64 on random tensors.
- attend_head with the 12-bit coefficients: one position gives the value row
  times its scale; equal keys give the mean of the values; against a float64
  softmax attention over the same int8 codes within the coefficients' error;
  the exponent total of the aarch64 build's four lanes differs from a
  sequential total on a planted input.
- table_indices: every index below the slot count, depends only on the last
  `order` tokens, positions before the start read token 0.
- The probe heads: the online softmax equals a float64 softmax over every
  observed token's cells (pooled readout), and the head output is the
  projection of it plus the bias.
- Loading: depth outside the ladder and a truncated archive are refused."""
import numpy as np
import pytest

import numpy_needle3
import oracle
import rustyneedle_amd as rn
from rustyneedle_amd import needle3

GEOMETRY = needle3.NEEDLE3_SMALL


@pytest.fixture(scope="module")
def archive():
    return needle3.synthetic_archive(GEOMETRY)


def _cos(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def test_step_against_float64_model(archive):
    om = oracle.OracleNeedle3(archive)
    ref = numpy_needle3.Model(archive, om.active).session()
    s = om.session(64)
    tokens = rn.synth_tokens(7, "needle3.pin", GEOMETRY["vocab"], (24,))
    for i, t in enumerate(tokens):
        s.push(int(t))
        ref.push(int(t))
        h = s.hidden()
        assert _cos(h, ref.hidden) > 0.999, i
        assert np.linalg.norm(h - ref.hidden) < 0.05 * np.linalg.norm(ref.hidden), i
        cells = s.cells()
        for layer in range(cells.shape[0]):
            assert _cos(cells[layer], ref.cells[layer]) > 0.999, (i, layer)
    logits, want = s.logits(), ref.logits()
    assert _cos(logits, want) > 0.999
    assert np.argmax(logits) == np.argmax(want)


def test_step_model_detects_a_dropped_term(archive):
    """The float64 model itself is sensitive: without the engram or the conv
    taps it leaves the oracle's cosine bound."""
    om = oracle.OracleNeedle3(archive)
    s = om.session(64)
    ref = numpy_needle3.Model(archive, om.active)
    for e in ref.engrams:
        e["value"] = np.zeros_like(e["value"])
    r = ref.session()
    tokens = rn.synth_tokens(7, "needle3.pin", GEOMETRY["vocab"], (8,))
    worst = 1.0
    for t in tokens:
        s.push(int(t))
        r.push(int(t))
        worst = min(worst, _cos(s.hidden(), r.hidden))
    assert worst < 0.999


def _hadamard_tensors(rng, width, rank=8):
    return dict(d1=1 + 0.1 * rng.standard_normal(1024), d2=1 + 0.1 * rng.standard_normal(1024),
                b2=0.1 * rng.standard_normal(1024), d3=1 + 0.1 * rng.standard_normal(1024),
                d4=0.5 + 0.1 * rng.standard_normal(1024),
                factors=rng.standard_normal((6, 32, 32)) / np.sqrt(32),
                cond_v=0.05 * rng.standard_normal((width, rank)), cond_u=0.2 * rng.standard_normal((rank, 1024)))


def test_hadamard_identity_is_silu():
    width = 768
    t = dict(d1=np.ones(1024), d2=np.ones(1024), b2=np.zeros(1024), d3=np.ones(1024), d4=np.ones(1024),
             factors=np.stack([np.eye(32)] * 6), cond_v=np.zeros((width, 8)), cond_u=np.zeros((8, 1024)))
    perm = np.arange(1024)
    x = np.random.default_rng(1).normal(0, 2, width).astype(np.float32)
    got = oracle.n3_hadamard(t, perm, perm, x)
    want = np.array([oracle.silu(float(v)) for v in x], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("rank", [8, 5])
def test_hadamard_against_float64(rank):
    rng = np.random.default_rng(rank)
    width = 768
    t = _hadamard_tensors(rng, width, rank)
    p1, p2 = rng.permutation(1024), rng.permutation(1024)
    x = rng.normal(0, 1, width).astype(np.float32)
    got = oracle.n3_hadamard(t, p1, p2, x).astype(np.float64)
    t64 = {k: np.asarray(np.asarray(v, np.float32), np.float64) for k, v in t.items()}
    x64 = x.astype(np.float64)
    w = x64 @ t64["cond_v"]
    w = np.exp(w - w.max())
    w /= w.sum()
    mod = 1 + w @ t64["cond_u"]
    f = t64["factors"]
    kron = lambda v, a, b: (a.T @ (v.reshape(32, 32) @ b)).reshape(-1)  # noqa: E731
    pad = np.zeros(1024)
    pad[:width] = x64
    first = kron(pad * t64["d1"], f[0], f[1])
    z = t64["d2"] * mod * first[p1] + t64["b2"]
    second = kron(z / (1 + np.exp(-z)), f[2], f[3])
    want = (kron(second[p2] * t64["d3"], f[4], f[5]) * t64["d4"])[:width]
    assert np.max(np.abs(got - want)) < 1e-4 * np.max(np.abs(want))


def test_attend_single_position_and_equal_keys():
    rng = np.random.default_rng(2)
    q = rng.integers(-127, 128, 64).astype(np.int8)
    k = rng.integers(-127, 128, (1, 64)).astype(np.int8)
    v = rng.integers(-127, 128, (1, 64)).astype(np.int8)
    out = oracle.n3_attend_head(q, 0.01, k, [0.02], v, [0.03])
    # one position: weight 2047 (e = 1, c = value scale), out = code * 2047 * (scale / 2047)
    scale = np.float32(0.03) / np.float32(2047.0)
    want = (v[0].astype(np.float32) * np.float32(2047.0)) * scale
    assert np.array_equal(out.view(np.uint32), want.astype(np.float32).view(np.uint32))
    keys = np.tile(k, (9, 1))
    values = rng.integers(-127, 128, (9, 64)).astype(np.int8)
    out = oracle.n3_attend_head(q, 0.01, keys, np.full(9, 0.02), values, np.full(9, 0.03))
    mean = values.astype(np.float64).mean(axis=0) * 0.03
    assert np.max(np.abs(out - mean)) < 1e-6 + 2e-3 * np.abs(mean).max()


@pytest.mark.parametrize("count", [1, 3, 4, 61, 400])
def test_attend_against_float64(count):
    rng = np.random.default_rng(count)
    q = rng.integers(-127, 128, 64).astype(np.int8)
    k = rng.integers(-127, 128, (count, 64)).astype(np.int8)
    v = rng.integers(-127, 128, (count, 64)).astype(np.int8)
    ks = rng.uniform(0.005, 0.02, count).astype(np.float32)
    vs = rng.uniform(0.005, 0.02, count).astype(np.float32)
    qs = np.float32(0.01 / 8)
    out = oracle.n3_attend_head(q, qs, k, ks, v, vs).astype(np.float64)
    scores = (k.astype(np.float64) @ q.astype(np.float64)) * ks * float(qs)
    w = np.exp(scores - scores.max())
    w /= w.sum()
    want = w @ (v.astype(np.float64) * vs[:, None])
    # 12-bit coefficients: each weight within half a step of peak / 2047
    assert np.max(np.abs(out - want)) < 2e-3 * np.abs(want).max() + 1e-6


def test_attend_total_is_four_lanes():
    """Position p adds into lane p % 4; a sequential total rounds differently
    on this input (a large first exponent, then many small ones)."""
    count = 12
    q = np.zeros(64, np.int8)
    q[0] = 100
    k = np.zeros((count, 64), np.int8)
    k[0, 0] = 100
    k[1:, 0] = 36
    v = np.ones((count, 64), np.int8)
    ks = np.full(count, 0.01, np.float32)
    vs = np.full(count, 0.01, np.float32)
    out = oracle.n3_attend_head(q, np.float32(0.01), k, ks, v, vs)
    c = ((k[:, 0].astype(np.float32) * np.float32(100) * ks) * np.float32(0.01)).astype(np.float32)
    e = np.array([oracle.fast_exp(float(x - c.max())) for x in c], np.float32)
    lanes = [np.float32(0)] * 4
    for p in range(count):
        lanes[p % 4] = np.float32(lanes[p % 4] + e[p])
    four = np.float32(np.float32(lanes[0] + lanes[1]) + np.float32(lanes[2] + lanes[3]))
    seq = np.float32(0)
    for x in e:
        seq = np.float32(seq + x)
    assert four != seq
    cc = (e * vs).astype(np.float32)
    scale = np.float32(cc.max() / np.float32(2047.0))
    ratios = np.array([np.float32(x / scale) for x in cc], np.float64)
    assert not np.any(ratios - np.floor(ratios) == 0.5)
    wts = np.round(ratios)
    total = np.float32(np.float32(wts.sum()) * scale)
    assert out[0] == np.float32(total * np.float32(np.float32(1.0) / four))


def test_table_indices(archive):
    cfg = oracle.OracleNeedle3(archive).config
    rng = np.random.default_rng(4)
    tokens = rng.integers(0, GEOMETRY["vocab"], 40).astype(np.uint32)
    for position in range(40):
        idx = oracle.n3_table_indices(cfg, tokens, position)
        assert len(idx) == GEOMETRY["num_engram_tables"] and all(0 <= i < GEOMETRY["engram_slots"] for i in idx)
        changed = tokens.copy()
        if position >= 3:
            changed[position - 3] ^= 1  # outside every order (2 and 3)
            assert oracle.n3_table_indices(cfg, changed, position) == idx
        changed = tokens.copy()
        changed[position] ^= 1
        assert oracle.n3_table_indices(cfg, changed, position) != idx
    # before the start the hash reads token 0: the first positions equal those of
    # the same tokens after two zeros
    padded = np.concatenate([np.zeros(2, np.uint32), tokens]).astype(np.uint32)
    for position in range(3):
        assert oracle.n3_table_indices(cfg, tokens, position) == oracle.n3_table_indices(cfg, padded, position + 2)


def test_heads_against_float64(archive):
    om = oracle.OracleNeedle3(archive)
    s = om.session(64)
    ref = numpy_needle3.Model(archive, om.active)
    heads = _heads(archive, om.active)
    tokens = rn.synth_tokens(9, "needle3.heads", GEOMETRY["vocab"], (12,))
    history = []
    for t in tokens:
        s.push(int(t))
        history.append(s.cells().astype(np.float64))
    cells = np.array(history)  # [tokens][layers][d]
    for code, h in heads.items():
        k, width = h["k"], cells.shape[2]
        slots = cells.shape[1] * k
        readouts = np.empty((slots, width))
        for slot in range(slots):
            layer = slot // k
            scores = cells[:, layer] @ h["probes"][slot] / np.sqrt(width)
            w = np.exp(scores - scores.max())
            w /= w.sum()
            avg = w @ cells[:, layer]
            readouts[slot] = avg / np.sqrt(np.mean(avg * avg) + 1e-6) * h["gain"][slot]
        pooled = np.empty((h["queries"], width))
        for q in range(h["queries"]):
            w = readouts @ h["query"][q] / np.sqrt(width) + h["row_bias"][q]
            w = np.exp(w - w.max())
            w /= w.sum()
            pooled[q] = w @ readouts
        got = s.pooled_readout(code).reshape(pooled.shape)
        assert np.max(np.abs(got - pooled)) < 1e-4 * np.abs(pooled).max(), code
        out = s.head_output(code)
        want = h["proj"] @ pooled.reshape(-1) + h["bias"]
        assert np.max(np.abs(out - want)) < 2e-3 * (np.abs(want).max() + 1), code
    assert s.head_output(3) is None
    del ref


def _heads(archive, active):
    """The probe head tensors of the archive, densified with the float64
    model's reader, rows selected for the active layers (heads.rs:51-82)."""
    g, cb, recs = numpy_needle3._parse(archive)
    L = g["num_layers"]
    idx = next(i for i, r in enumerate(recs) if r["kind"] == 1 and len(r["shape"]) == 1 and r["shape"][0] == 2
               and i > 10)
    codes = [int(round(c)) for c in numpy_needle3._floats(recs[idx])]
    out, at = {}, idx + 1
    rows = [0] + [a + 1 for a in active]
    for code in codes:
        probes = numpy_needle3._dense(recs[at], cb)
        gain = numpy_needle3._floats(recs[at + 1])
        query = numpy_needle3._dense(recs[at + 2], cb)
        row_bias = numpy_needle3._floats(recs[at + 3]).reshape(query.shape[0], -1)
        proj = numpy_needle3._dense(recs[at + 4], cb)
        bias = numpy_needle3._floats(recs[at + 5])
        at += 6 + (code == 3)
        k = probes.shape[0] // (L + 1)
        sel = [r * k + p for r in rows for p in range(k)]
        out[code] = dict(k=k, probes=probes[sel], gain=gain[sel], query=query, row_bias=row_bias[:, sel], proj=proj,
                         bias=bias, queries=query.shape[0])
    return out


def test_loading_errors(archive):
    with pytest.raises(ValueError):
        oracle.OracleNeedle3(archive, depth=1)
    with pytest.raises(ValueError):
        oracle.OracleNeedle3(archive[:-200])
    assert oracle.OracleNeedle3(archive, depth=2).active == [0, 3]


def test_prefill_of_float_path_matrices_differs_from_pushes():
    """Session::feed runs chunks of at least four tokens as prefills
    (session.rs:56-70), whose projections and engram products go through
    multiply_batch; for 1- and 3-bit matrices that is the float tile
    (matrix.rs:356-378), which rounds differently from the vector product of a
    push. With 3-bit projections and engram matrices the oracle's feed must
    therefore differ from pushing the same tokens, while with the default
    (2-bit) layout the two are equal bit for bit; a feed of fewer than four
    tokens is pushes in both."""
    from rustyneedle_amd import needle3
    tokens = rn.synth_tokens(3, "needle3.tokens", needle3.NEEDLE3_SMALL["vocab"], (21,))
    for bits, differs in ((dict(needle3.BITS, projection=3, engram=3), True), (needle3.BITS, False)):
        om = oracle.OracleNeedle3(needle3.synthetic_archive(needle3.NEEDLE3_SMALL, bits=bits))
        fed, pushed = om.session(64), om.session(64)
        fed.feed(tokens)
        for t in tokens:
            pushed.push(int(t))
        same = np.array_equal(fed.logits().view(np.uint32), pushed.logits().view(np.uint32))
        assert same != differs, bits
        short_fed, short_pushed = om.session(8), om.session(8)
        short_fed.feed(tokens[:3])
        for t in tokens[:3]:
            short_pushed.push(int(t))
        assert np.array_equal(short_fed.hidden().view(np.uint32), short_pushed.hidden().view(np.uint32))

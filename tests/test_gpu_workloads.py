"""The prefill and batched-decode workloads at full size against the oracle.

The model is the 20-layer decoder (d_model 512, 8 heads of 64, FFN 2048,
vocab 8192, int8 codes with per-32 scales, fp16 cache) the benchmark runs,
with the benchmark's own seeded inputs:
- prefill: one 256-token `feed` of ids U{0..8191} into an empty session
  (crates/model/src/session.rs:56-70, crates/model/src/prefill.rs:10-99),
  compared bit for bit (hidden state, logits, the whole cache) with the
  oracle and with 256 single-token pushes on the GPU;
- batched decode: 64 sequences with caches of U[32, 512] positions, 32 greedy
  steps (crates/generate/src/generator.rs:199-265 per sequence), every id,
  every sequence's final logits and a sample of the caches compared bit for
  bit with the oracle run one sequence at a time.
"""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import oracle
import rustyneedle_amd as rn

pytestmark = pytest.mark.gpu

# oracle sessions run concurrently, one thread each (ctypes releases the GIL)
WORKERS = 12


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def needle():
    cfg = dict(rn.NEEDLE_DECODER)
    w = rn.synthetic_weights(cfg)
    return cfg, rn.Model(cfg, w), oracle.OracleModel(cfg, w)


def test_prefill_256_tokens_full_model(needle):
    cfg, gm, om = needle
    tokens = rn.synth_tokens(rn.SEED, "prefill.tokens", cfg["vocab"], 256)
    gs = gm.session(256)
    gs.feed(tokens)
    oracle.set_threads(WORKERS)
    try:
        os_ = om.session(256)
        os_.feed(tokens)
    finally:
        oracle.set_threads(1)
    assert len(gs) == os_.length == 256
    assert np.array_equal(_bits(gs.hidden()), _bits(os_.hidden))
    assert np.array_equal(_bits(gs.logits()), _bits(os_.logits()))
    k, v = gs.get_cache()
    assert np.array_equal(k.view(np.uint16), os_.keys)
    assert np.array_equal(v.view(np.uint16), os_.values)
    # the same positions one token at a time (the decode kernels) on the GPU
    gp = gm.session(256)
    for t in tokens:
        gp.push(int(t))
    assert np.array_equal(_bits(gp.hidden()), _bits(os_.hidden))
    pk, pv = gp.get_cache()
    assert np.array_equal(pk.view(np.uint16), os_.keys)
    assert np.array_equal(pv.view(np.uint16), os_.values)


def test_batch64_ragged_32_steps_full_model(needle):
    cfg, gm, om = needle
    count, steps = 64, 32
    lengths = (rn.synth_tokens(rn.SEED, "batch.lengths", 481, count) + 32).astype(np.int32)
    first = rn.synth_tokens(rn.SEED, "batch.first", cfg["vocab"], count)
    assert lengths.min() >= 32 and lengths.max() <= 512
    with ThreadPoolExecutor(WORKERS) as ex:
        caches = list(ex.map(lambda i: rn.synthetic_cache(cfg, int(lengths[i]), f"batch.{i}"), range(count)))
    b = rn.Batch(gm, count, int(lengths.max()) + steps)
    for i in range(count):
        b.set_cache(i, *caches[i])
    ids = b.decode_greedy(first, steps)
    logits = b.logits()

    oracle.set_threads(1)

    def run(i):
        o = om.session(int(lengths[i]) + steps)
        o.set_cache(*caches[i])
        return o.greedy(int(first[i]), steps), o.logits(), o

    with ThreadPoolExecutor(WORKERS) as ex:
        ref = list(ex.map(run, range(count)))
    bad = [i for i in range(count) if ids[i].tolist() != ref[i][0].tolist()]
    assert not bad, f"sequences whose greedy ids differ from the oracle: {bad}"
    bad = [i for i in range(count) if not np.array_equal(_bits(logits[i]), _bits(ref[i][1]))]
    assert not bad, f"sequences whose final logits differ from the oracle: {bad}"
    # caches: the shortest, the longest and two in between, all positions
    for i in {int(np.argmin(lengths)), int(np.argmax(lengths)), 0, count - 1}:
        n = int(lengths[i]) + steps
        k, v = b.get_cache(i, n)
        o = ref[i][2]
        assert np.array_equal(k.view(np.uint16), o.keys[:, :, :n]), i
        assert np.array_equal(v.view(np.uint16), o.values[:, :, :n]), i


def test_needle3_full_size_feed_equals_pushes(monkeypatch):
    """The Needle 3 block at its documented shape (d_model 768, 20 layers, 12
    heads over 4 kv heads, four lanes, two engram sites, a 1024 window with
    four global layers): a 300-token feed (a 256-token run, then 44) leaves
    the same state, bit for bit, as 300 pushes (each push is pinned to the
    oracle in test_gpu_needle3.py); then 8 greedy tokens from both."""
    from rustyneedle_amd import needle3
    monkeypatch.delenv("RN_N3_PATH", raising=False)
    monkeypatch.delenv("RN_N3_FEED_CHUNK", raising=False)
    g = needle3.NEEDLE3
    model = needle3.Model(needle3.synthetic_archive(g))
    tokens = rn.synth_tokens(rn.SEED, "needle3.feed", g["vocab"], (300,))
    fed, pushed = model.session(320), model.session(320)
    print("needle3 full-size feed of 300 tokens", flush=True)
    fed.feed(tokens)
    print("needle3 full-size 300 pushes", flush=True)
    for t in tokens:
        pushed.push(int(t))
    bits = lambda a: np.ascontiguousarray(a, np.float32).view(np.uint32)
    assert np.array_equal(bits(fed.hidden()), bits(pushed.hidden()))
    assert np.array_equal(bits(fed.cells()), bits(pushed.cells()))
    assert np.array_equal(bits(fed.logits()), bits(pushed.logits()))
    for code in (1, 2):
        assert np.array_equal(bits(fed.pooled_readout(code)), bits(pushed.pooled_readout(code))), code
    for layer in (0, 1, 10, 19):
        for a, b in zip(fed.cache(layer), pushed.cache(layer)):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), layer
    assert fed.decode_greedy(7, 8).tolist() == pushed.decode_greedy(7, 8).tolist()


@pytest.mark.timeout(600)
def test_needle3_documented_geometry_against_the_oracle(monkeypatch):
    """The Needle 3 block at its documented shape (d_model 768, 20 layers, 12
    heads over 4 kv heads, four lanes, two engram sites at layers 1 and 10, a
    1024-token window with layers 4, 9, 14 and 19 global) against the oracle,
    bit for bit: a 1040-token feed (batched runs; the last 16 positions are past
    the window of the 16 non-global layers, attention.rs:171-177), then 8 greedy
    tokens (session.rs:76-148 per push). Compared: hidden state, cells, logits,
    both probe heads' pooled readouts and outputs, and the int8 caches (codes and
    scales) of layers 0, 1, 4, 10 and 19, after the feed and after the tokens."""
    from rustyneedle_amd import needle3
    monkeypatch.delenv("RN_N3_PATH", raising=False)
    monkeypatch.delenv("RN_N3_FEED_CHUNK", raising=False)
    g = needle3.NEEDLE3
    archive = needle3.synthetic_archive(g)
    gm, om = needle3.Model(archive), oracle.OracleNeedle3(archive)
    tokens = rn.synth_tokens(rn.SEED, "needle3.window", g["vocab"], (1040,))
    gs, os_ = gm.session(1056), om.session(1056)

    def oracle_feed():
        for a in range(0, tokens.size, 130):
            print(f"needle3 documented geometry: oracle pushes {a}..{min(a + 130, tokens.size)}", flush=True)
            os_.feed(tokens[a:a + 130])

    with ThreadPoolExecutor(1) as pool:
        done = pool.submit(oracle_feed)
        print("needle3 documented geometry: device feed of 1040 tokens", flush=True)
        gs.feed(tokens)
        done.result()

    def compare(label):
        assert len(gs) == len(os_), label
        assert np.array_equal(_bits(gs.hidden()), _bits(os_.hidden())), f"hidden {label}"
        assert np.array_equal(_bits(gs.cells()), _bits(os_.cells())), f"cells {label}"
        assert np.array_equal(_bits(gs.logits()), _bits(os_.logits())), f"logits {label}"
        for code in (1, 2):
            assert np.array_equal(_bits(gs.pooled_readout(code)), _bits(os_.pooled_readout(code))), (label, code)
            assert np.array_equal(_bits(gs.head_output(code)), _bits(os_.head_output(code))), (label, code)
        for layer in (0, 1, 4, 10, 19):
            for a, b in zip(gs.cache(layer), os_.cache(layer)):
                assert a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8)), (label, layer)

    compare("after the 1040-token feed")
    print("needle3 documented geometry: 8 greedy tokens", flush=True)
    ids = gs.decode_greedy(7, 8)
    assert ids.tolist() == os_.greedy(7, 8).tolist()
    compare("after 8 greedy tokens")

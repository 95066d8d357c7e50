"""The multi-lane hyper-connection (crates/model/src/lanes.rs).

Oracle pins (CPU): unit_rms against float64 (ops.rs:60-66); Sinkhorn rows and
columns sum to one after its iterations, its fixed point for a constant input
is uniform, and a float64 Sinkhorn agrees; combine_into against a float64
restatement. GPU: route and combine bit for bit against the oracle (the gates
and Sinkhorn call the device's restatement of the C library's expf, which the
reference's f32::exp and the oracle call)."""
import numpy as np
import pytest

import oracle
import rustyneedle_amd as rn

LANES, WIDTH, LAYERS = 4, 128, 2


def test_unit_rms_against_float64():
    x = np.random.default_rng(1).normal(0, 2, 512).astype(np.float32)
    got = oracle.unit_rms(x)
    x64 = x.astype(np.float64)
    assert np.max(np.abs(got - x64 / np.sqrt(np.mean(x64 ** 2) + 1e-6))) < 1e-6 * np.abs(got).max()


def test_sinkhorn_is_doubly_stochastic():
    m = np.random.default_rng(2).normal(0, 1, 16).astype(np.float32)
    s = oracle.sinkhorn(m).reshape(4, 4)
    assert np.max(np.abs(s.sum(axis=0) - 1)) < 1e-6 and np.max(np.abs(s.sum(axis=1) - 1)) < 1e-4
    assert np.allclose(oracle.sinkhorn(np.full(16, 3.0, np.float32)), 0.25, atol=1e-7)
    e = np.exp(m.astype(np.float64).reshape(4, 4) - m.reshape(4, 4).max(axis=1, keepdims=True))
    for _ in range(20):
        e /= e.sum(axis=1, keepdims=True)
        e /= e.sum(axis=0, keepdims=True)
    assert np.max(np.abs(s - e)) < 1e-5


def test_combine_against_float64():
    rng = np.random.default_rng(3)
    post, res = rng.random(LANES).astype(np.float32), rng.random((LANES, LANES)).astype(np.float32)
    stream, delta = rng.normal(0, 1, (LANES, WIDTH)).astype(np.float32), rng.normal(0, 1, WIDTH).astype(np.float32)
    got = oracle.lanes_combine(LANES, WIDTH, post, res, stream, delta)
    want = res.astype(np.float64) @ stream.astype(np.float64) + post[:, None].astype(np.float64) * delta[None, :]
    assert np.max(np.abs(got - want)) < 1e-5


def _setup(bits=4):
    rng = np.random.default_rng(4)
    t = dict(a_pre=rng.normal(0, 1, LAYERS), a_post=rng.normal(0, 1, LAYERS), a_res=rng.normal(0, 1, LAYERS),
             b_pre=rng.normal(0, 1, LAYERS * LANES), b_post=rng.normal(0, 1, LAYERS * LANES),
             b_res=rng.normal(0, 1, LAYERS * LANES * LANES))
    t = {k: v.astype(np.float32) for k, v in t.items()}
    cb = rn.synthetic_codebook(128)
    rows = (LAYERS * LANES, LAYERS * LANES, LAYERS * LANES * LANES)
    blobs = [rn.synthetic_codebook_blob(r, LANES * WIDTH, 128, bits, seed=10 + i) for i, r in enumerate(rows)]
    return t, cb, rows, blobs


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [2, 4, 5])
def test_route_and_combine_on_the_gpu(bits):
    """Every output bit for 2-bit (panel form), 4-bit and ternary (plane form)
    routing matrices, at layer 0 and at layer 1 (rows past the first layer's)."""
    t, cb, rows, blobs = _setup(bits)
    gphis = [rn.CodebookMatrix(b, r, LANES * WIDTH, 128, bits, cb) for b, r in zip(blobs, rows)]
    ophis = [oracle.OracleCodebookMatrix(b, r, LANES * WIDTH, 128, bits, cb) for b, r in zip(blobs, rows)]
    lanes = rn.Lanes(LANES, WIDTH, LAYERS, t["a_pre"], t["a_post"], t["a_res"], t["b_pre"], t["b_post"], t["b_res"],
                     *gphis)
    stream = np.random.default_rng(5).normal(0, 1, (LANES, WIDTH)).astype(np.float32)
    for layer, slot in ((0, 0), (1, 6)):
        gi, gp, gr = lanes.route(layer, slot, stream)
        oi, op, orr = oracle.lanes_route(LANES, WIDTH, layer, slot, t, stream, ophis)
        for g, o in ((gi, oi), (gp, op), (gr, orr)):
            assert np.array_equal(g.view(np.uint32), o.view(np.uint32))
        delta = np.random.default_rng(layer).normal(0, 1, WIDTH).astype(np.float32)
        got = lanes.combine(gp, gr, stream, delta)
        want = oracle.lanes_combine(LANES, WIDTH, gp, gr, stream, delta)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))

"""The grammar-constrained choice (generator.rs:99-117, 147-194) on the GPU against
the oracle, bit for bit, through the C ABI."""
import numpy as np
import pytest

import oracle
import rustyneedle_amd as rn

pytestmark = pytest.mark.gpu


def _check(logits, mask, token=-1):
    got = rn.choose_allowed(logits, mask, token)
    if token < 0:
        want = oracle.choose_allowed(logits, mask)
        assert got[1] == (oracle.argmax_allowed(logits, mask) >= 0)
    else:
        want = (token,) + oracle.allowed_statistics(logits, mask, token)
    assert got[0] == want[0]
    assert np.array_equal(np.float32([got[2], got[3]]).view(np.uint32), np.float32([want[1], want[2]]).view(np.uint32))
    return got


@pytest.mark.parametrize("n,density", [(8192, 0.5), (8192, 0.01), (10000, 0.3), (5000, 0.9), (1, 1.0), (4097, 0.2)])
def test_random_masks(n, density):
    rng = np.random.default_rng(n)
    logits = rng.normal(0, 4, n).astype(np.float32)
    mask = (rng.random(n) < density).astype(np.uint8)
    _check(logits, mask)
    _check(logits, np.ones(n, np.uint8))
    _check(logits, mask, token=n // 2)


def test_edges():
    rng = np.random.default_rng(1)
    v = rng.normal(0, 1, 8192).astype(np.float32)
    none = np.zeros(8192, np.uint8)
    _check(v, none)                                   # nothing allowed: argmax, statistics of it
    one = none.copy()
    one[4321] = 1
    assert _check(v, one)[0] == 4321
    ties = np.zeros(8192, np.float32)
    assert _check(ties, np.ones(8192, np.uint8))[0] == 0
    w = v.copy()
    w[[10, 20]] = np.nan                              # NaN as the first allowed value wins
    m = none.copy()
    m[[10, 20, 30]] = 1
    assert _check(w, m)[0] == 10
    w2 = v.copy()
    w2[20] = np.nan                                   # a later NaN never wins
    assert _check(w2, m)[0] in (10, 30)
    x = v.copy()
    x[0] = np.nan                                     # argmax fallback with a NaN at index 0
    assert _check(x, none)[0] == 0
    y = v.copy()
    y[5] = np.inf
    _check(y, np.ones(8192, np.uint8))
    _check(np.full(8192, -np.inf, np.float32), one)


def test_session_choice_matches_the_oracle(tiny, tiny_config):
    gm, om = tiny
    gs, os_ = gm.session(16), om.session(16)
    rng = np.random.default_rng(5)
    for tok in (3, 999, 12):
        gs.push(tok)
        os_.push(tok)
        mask = (rng.random(tiny_config["vocab"]) < 0.1).astype(np.uint8)
        token, constrained, p, m = gs.choose_allowed(mask)
        want = oracle.choose_allowed(os_.logits(), mask)
        assert (token, constrained) == (want[0], True)
        assert np.array_equal(np.float32([p, m]).view(np.uint32), np.float32(want[1:]).view(np.uint32))
    with pytest.raises(rn.RnError):
        gm.session(4).choose_allowed(np.ones(tiny_config["vocab"], np.uint8))  # nothing pushed yet


@pytest.fixture(scope="module")
def tiny(tiny_config, tiny_weights):
    return rn.Model(tiny_config, tiny_weights), oracle.OracleModel(tiny_config, tiny_weights)

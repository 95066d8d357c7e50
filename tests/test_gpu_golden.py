"""The HIP path against the committed golden fixtures (through the C ABI)."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_golden  # noqa: E402

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(HERE, "golden")


def test_gemv_fixture_on_gpu():
    import rustyneedle_amd as rn
    g = np.load(os.path.join(GOLDEN, "gemv_2048x512.npz"), allow_pickle=False)
    W, sW, x = make_golden.gemv_inputs()
    m = rn.QuantisedMatrix(W, sW)
    y, acc = m.multiply_vector_host(x, with_acc=True)
    assert np.array_equal(acc.reshape(2048, 16), g["acc"])
    assert np.array_equal(y.view(np.uint32), g["y"].view(np.uint32))


def test_decode_fixture_on_gpu():
    import rustyneedle_amd as rn
    g = np.load(os.path.join(GOLDEN, "decode_20l_16.npz"), allow_pickle=False)
    cfg, _, keys, values, first = make_golden.decode_inputs()
    model = rn.Model(cfg, seed=rn.SEED)
    s = model.session(make_golden.CONTEXT + make_golden.STEPS)
    s.set_cache(keys, values)
    ids = s.decode_greedy(first, make_golden.STEPS)
    assert ids.tolist() == g["ids"].tolist()
    s.truncate(make_golden.CONTEXT)
    s.push(first)
    assert np.array_equal(s.logits().view(np.uint32), g["logits0"].view(np.uint32))

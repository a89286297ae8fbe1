"""The persistent single-launch decode step against the per-kernel path and
the oracle: identical logits bits, KV rows and greedy tokens."""
import os

import numpy as np
import pytest

from funasrnet_amd import model

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def backend():
    from funasrnet_amd.hip import HipBackend
    b = HipBackend(0)
    yield b
    b.close()


def _decoder(backend, weights, persistent, capacity):
    from funasrnet_amd.hip import HipDecoder
    old = os.environ.get("FAH_PERSISTENT")
    os.environ["FAH_PERSISTENT"] = "1" if persistent else "0"
    try:
        return HipDecoder(backend, weights, capacity=capacity)
    finally:
        if old is None:
            del os.environ["FAH_PERSISTENT"]
        else:
            os.environ["FAH_PERSISTENT"] = old


@pytest.mark.parametrize("shape", ["small", "qwen3"])
def test_persistent_matches_graph_path(backend, oracle_lib, shape):
    cfg = model.small_config(layers=2) if shape == "small" else model.QWEN3_0_6B
    w = model.synthetic(cfg, seed=7)
    frames = 12 if shape == "small" else 150
    steps = 10 if shape == "small" else 24
    prefix = np.random.default_rng(11).standard_normal((frames, cfg.width)).astype(np.float32)
    fast = _decoder(backend, w, True, 1024)
    slow = _decoder(backend, w, False, 1024)
    try:
        assert fast.persistent and not slow.persistent
        lf = fast.decode(prefix, frames)
        ls = slow.decode(prefix, frames)
        assert np.array_equal(lf.view(np.uint32), ls.view(np.uint32))
        assert fast.greedy() == slow.greedy() == oracle_lib.greedy(ls)
        tf = fast.generate(steps)
        ts = slow.generate(steps)
        assert tf.tolist() == ts.tolist()
        for layer in (0, cfg.layers - 1):
            kf, vf = fast.kv_read(layer, frames + steps)
            ks, vs = slow.kv_read(layer, frames + steps)
            assert np.array_equal(kf.view(np.uint16), ks.view(np.uint16))
            assert np.array_equal(vf.view(np.uint16), vs.view(np.uint16))
        x = fast.embed([int(tf[-1])])
        lf = fast.decode(x, 1)
        ls = slow.decode(x, 1)
        assert np.array_equal(lf.view(np.uint32), ls.view(np.uint32))
    finally:
        fast.close()
        slow.close()


def test_persistent_against_oracle_tokens(backend, oracle_lib):
    w = model.synthetic(model.small_config(layers=2), seed=8)
    prefix = np.random.default_rng(5).standard_normal((9, w.config.width)).astype(np.float32)
    fast = _decoder(backend, w, True, 256)
    ref = oracle_lib.Decoder(w, capacity=256)
    try:
        lg = fast.decode(prefix, 9)
        lr = ref.decode(prefix, 9)
        assert np.abs(lg - lr).max() <= 1e-2
        toks = fast.generate(20)
        expected = []
        for _ in range(20):
            t = oracle_lib.greedy(lr)
            expected.append(t)
            lr = ref.decode(ref.embed([t]), 1)
        assert toks.tolist() == expected
    finally:
        fast.close()
        ref.close()

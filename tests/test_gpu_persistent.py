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


def _decoder(backend, weights, persistent, capacity, local_l2=None, long_from=None, persistent_positions=None):
    from funasrnet_amd.hip import HipDecoder
    env = {"FAH_PERSISTENT": "1" if persistent else "0"}
    if local_l2 is not None:
        env["FAH_LOCAL_L2"] = "1" if local_l2 else "0"
    if long_from is not None:
        env["FAH_LONG_FROM"] = str(long_from)
    if persistent_positions is not None:
        env["FAH_PERSISTENT_POSITIONS"] = str(persistent_positions)
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return HipDecoder(backend, weights, capacity=capacity)
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


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


@pytest.mark.parametrize("shape,positions,persistent_positions",
                         [("small", 4096, None), ("qwen3", 4096, None), ("qwen3", 2048, 2052)])
def test_long_cache_matches_graph_path(backend, oracle_lib, shape, positions, persistent_positions):
    """A cache pre-filled with F16 N(0,1) rows in every layer: the persistent
    kernel's long-cache attention (scores on the projection workgroups, the
    value sums on value workgroups from the published probabilities; at
    2048 positions with FAH_PERSISTENT_POSITIONS=2052, so that the greedy
    steps cross over to the per-kernel path) and the per-kernel path give
    identical logits bits, K/V rows and tokens, and match the oracle (the
    full-size shape too, 8 greedy steps)."""
    cfg = model.small_config(layers=2) if shape == "small" else model.QWEN3_0_6B
    w = model.synthetic(cfg, seed=12)
    capacity, steps = positions + 128, 8
    rng = np.random.default_rng(13)
    kv = [(rng.standard_normal((positions, cfg.kv_width)).astype(np.float16),
           rng.standard_normal((positions, cfg.kv_width)).astype(np.float16)) for _ in range(cfg.layers)]
    x = rng.standard_normal((1, cfg.width)).astype(np.float32)
    fast = _decoder(backend, w, True, capacity, persistent_positions=persistent_positions)
    slow = _decoder(backend, w, False, capacity)
    try:
        assert fast.persistent and not slow.persistent
        for d in (fast, slow):
            for layer, (k, v) in enumerate(kv):
                d.kv_write(layer, k, v)
            d.set_position(positions)
        print(f"long cache {shape} positions={positions}", flush=True)
        lf = fast.decode(x, 1)
        ls = slow.decode(x, 1)
        assert np.array_equal(lf.view(np.uint32), ls.view(np.uint32))
        tf = fast.generate(steps)
        ts = slow.generate(steps)
        assert tf.tolist() == ts.tolist()
        for layer in (0, cfg.layers - 1):
            kf, vf = fast.kv_read(layer, positions + 1 + steps)
            ks, vs = slow.kv_read(layer, positions + 1 + steps)
            assert np.array_equal(kf.view(np.uint16), ks.view(np.uint16))
            assert np.array_equal(vf.view(np.uint16), vs.view(np.uint16))
            assert np.array_equal(kf[:positions * cfg.kv_width].view(np.uint16), kv[layer][0].view(np.uint16).ravel())
        ref = oracle_lib.Decoder(w, capacity=capacity)
        try:
            for layer, (k, v) in enumerate(kv):
                ref.set_kv(layer, k.astype(np.float32), v.astype(np.float32))
            ref.set_position(positions)
            lr = ref.decode(x, 1)
            assert np.abs(lf.astype(np.float64) - lr).max() <= 1e-2
            assert np.array_equal(lf.view(np.uint32), lr.view(np.uint32))
            expected = []
            for _ in range(steps):
                t = oracle_lib.greedy(lr)
                expected.append(t)
                lr = ref.decode(ref.embed([t]), 1)
            assert tf.tolist() == expected
            for layer in (0, cfg.layers - 1):
                kf, vf = fast.kv_read(layer, positions + 1 + steps)
                ko, vo = ref.kv(layer)
                assert np.array_equal(kf.astype(np.float32), ko.reshape(kf.shape)), layer
                assert np.array_equal(vf.astype(np.float32), vo.reshape(vf.shape)), layer
        finally:
            ref.close()
    finally:
        fast.close()
        slow.close()


@pytest.mark.parametrize("shape", ["small", "qwen3"])
def test_steps_across_the_persistent_range(backend, shape):
    """The persistent kernel's attention workgroups hold every earlier K/V
    row below position 483 and take the long-cache attention from there on:
    generating across that boundary (from a 466-row prefix), and decoding
    single rows after it, matches a decoder that never used the persistent
    kernel."""
    cfg = model.small_config(layers=2) if shape == "small" else model.QWEN3_0_6B
    w = model.synthetic(cfg, seed=15)
    prefix = np.random.default_rng(16).standard_normal((466, cfg.width)).astype(np.float32)
    fast = _decoder(backend, w, True, 512)
    slow = _decoder(backend, w, False, 512)
    try:
        assert fast.persistent and not slow.persistent
        print(f"persistent boundary {shape}", flush=True)
        lf = fast.decode(prefix, 466)
        ls = slow.decode(prefix, 466)
        assert np.array_equal(lf.view(np.uint32), ls.view(np.uint32))
        tf = fast.generate(30)
        ts = slow.generate(30)
        assert tf.tolist() == ts.tolist()
        x = fast.embed([int(tf[-1])])
        lf = fast.decode(x, 1)
        ls = slow.decode(x, 1)
        assert np.array_equal(lf.view(np.uint32), ls.view(np.uint32))
        for layer in (0, cfg.layers - 1):
            kf, vf = fast.kv_read(layer, 497)
            ks, vs = slow.kv_read(layer, 497)
            assert np.array_equal(kf.view(np.uint16), ks.view(np.uint16))
            assert np.array_equal(vf.view(np.uint16), vs.view(np.uint16))
        # Back below the boundary: the persistent kernel again.
        fast.set_position(200)
        slow.set_position(200)
        lf = fast.decode(x, 1)
        ls = slow.decode(x, 1)
        assert np.array_equal(lf.view(np.uint32), ls.view(np.uint32))
        assert fast.generate(5).tolist() == slow.generate(5).tolist()
    finally:
        fast.close()
        slow.close()


def test_persistent_after_long_prefix_matches_oracle(backend, oracle_lib):
    """A 375-row prefix, then 16 greedy steps on the persistent
    kernel (positions 375-390, past the V rows its attention workgroups
    once held): every token equals the oracle's and the next row's logits
    are bit-identical to the oracle's."""
    cfg = model.QWEN3_0_6B
    w = model.synthetic(cfg, seed=21)
    frames, steps = 375, 16
    prefix = np.random.default_rng(22).standard_normal((frames, cfg.width)).astype(np.float32)
    fast = _decoder(backend, w, True, 512)
    ref = oracle_lib.Decoder(w, capacity=512)
    try:
        assert fast.persistent
        print(f"persistent after {frames}-row prefix", flush=True)
        lf = fast.decode(prefix, frames)
        lr = ref.decode(prefix, frames)
        assert np.array_equal(lf.view(np.uint32), lr.view(np.uint32))
        toks = fast.generate(steps)
        expected = []
        for _ in range(steps):
            t = oracle_lib.greedy(lr)
            expected.append(t)
            lr = ref.decode(ref.embed([t]), 1)
        assert toks.tolist() == expected
        t = int(toks[-1])
        lf = fast.decode(fast.embed([t]), 1)
        lr = ref.decode(ref.embed([t]), 1)
        assert np.array_equal(lf.view(np.uint32), lr.view(np.uint32))
    finally:
        fast.close()
        ref.close()


@pytest.mark.parametrize("shape,local_l2", [("small", True), ("qwen3", True), ("qwen3", False)])
def test_long_attention_at_every_position_matches_oracle(backend, oracle_lib, shape, local_l2):
    """FAH_LONG_FROM=0: the long-cache attention (scores by the projection
    workgroups, V rows through the ring) at every position. From an empty
    cache, 40 single-row steps (shares of the earlier positions empty below
    30, partial ring segments and padded score chunks), then a 150-row
    prefix and 16 greedy steps: logits bits and tokens equal the oracle's."""
    cfg = model.small_config(layers=2) if shape == "small" else model.QWEN3_0_6B
    w = model.synthetic(cfg, seed=31)
    rng = np.random.default_rng(32)
    fast = _decoder(backend, w, True, 256, local_l2=local_l2, long_from=0)
    ref = oracle_lib.Decoder(w, capacity=256)
    try:
        assert fast.persistent
        print(f"long attention everywhere {shape} local_l2={local_l2}", flush=True)
        for step in range(40):
            x = rng.standard_normal((1, cfg.width)).astype(np.float32)
            lf = fast.decode(x, 1)
            lr = ref.decode(x, 1)
            assert np.array_equal(lf.view(np.uint32), lr.view(np.uint32)), step
        for layer in (0, cfg.layers - 1):
            kf, vf = fast.kv_read(layer, 40)
            ko, vo = ref.kv(layer)
            assert np.array_equal(kf.astype(np.float32), ko), layer
            assert np.array_equal(vf.astype(np.float32), vo), layer
        fast.set_position(0)
        ref.set_position(0)
        prefix = rng.standard_normal((150, cfg.width)).astype(np.float32)
        lf = fast.decode(prefix, 150)
        lr = ref.decode(prefix, 150)
        assert np.array_equal(lf.view(np.uint32), lr.view(np.uint32))
        toks = fast.generate(16)
        expected = []
        for _ in range(16):
            t = oracle_lib.greedy(lr)
            expected.append(t)
            lr = ref.decode(ref.embed([t]), 1)
        assert toks.tolist() == expected
    finally:
        fast.close()
        ref.close()


@pytest.mark.parametrize("persistent,long_from", [(True, None), (True, 0), (False, None)])
def test_peaked_attention_matches_oracle(backend, oracle_lib, persistent, long_from):
    """K rows scaled by 24 give scores far apart, so many softmax numerators
    fall below 2^-17 and the denominator takes the reference's sequential
    order (not the exact wave-tree sum that flatter scores allow): logits
    bits equal the oracle's over 6 steps at 300 cached positions, with the
    persistent kernel's short-cache attention, its long-cache one
    (FAH_LONG_FROM=0) and the multi-kernel step."""
    cfg = model.small_config(layers=2)
    w = model.synthetic(cfg, seed=41)
    positions, capacity = 300, 512
    rng = np.random.default_rng(42)
    kv = [((24.0 * rng.standard_normal((positions, cfg.kv_width))).astype(np.float16),
           rng.standard_normal((positions, cfg.kv_width)).astype(np.float16)) for _ in range(cfg.layers)]
    fast = _decoder(backend, w, persistent, capacity, long_from=long_from)
    ref = oracle_lib.Decoder(w, capacity=capacity)
    try:
        assert bool(fast.persistent) == persistent
        print(f"peaked attention persistent={persistent} long_from={long_from}", flush=True)
        for layer, (k, v) in enumerate(kv):
            fast.kv_write(layer, k, v)
            ref.set_kv(layer, k.astype(np.float32), v.astype(np.float32))
        fast.set_position(positions)
        ref.set_position(positions)
        for step in range(6):
            x = rng.standard_normal((1, cfg.width)).astype(np.float32)
            lf = fast.decode(x, 1)
            lr = ref.decode(x, 1)
            assert np.array_equal(lf.view(np.uint32), lr.view(np.uint32)), step
    finally:
        fast.close()
        ref.close()


@pytest.mark.parametrize("shape", ["small", "qwen3"])
def test_persistent_without_xcd_roles_matches_graph_path(backend, oracle_lib, shape):
    """FAH_LOCAL_L2=0: roles by workgroup index, every hand-over through
    device-scope stores (the mode a launch falls back to when the XCD
    dealing it relies on is broken) gives the same bits."""
    from funasrnet_amd.hip import load
    cfg = model.small_config(layers=2) if shape == "small" else model.QWEN3_0_6B
    w = model.synthetic(cfg, seed=5)
    frames = 12 if shape == "small" else 150
    prefix = np.random.default_rng(13).standard_normal((frames, cfg.width)).astype(np.float32)
    plain = _decoder(backend, w, True, 1024, local_l2=False)
    slow = _decoder(backend, w, False, 1024)
    try:
        assert load().fah_decoder_persistent(plain.handle) == 1
        lp = plain.decode(prefix, frames)
        ls = slow.decode(prefix, frames)
        assert np.array_equal(lp.view(np.uint32), ls.view(np.uint32))
        assert plain.greedy() == slow.greedy() == oracle_lib.greedy(ls)
        assert plain.generate(8).tolist() == slow.generate(8).tolist()
    finally:
        plain.close()
        slow.close()


@pytest.mark.parametrize("bad", ["nan", "inf", "huge"])
def test_persistent_non_finite_rows_match_graph_path(backend, oracle_lib, bad):
    """Rows with a NaN, an infinity or values near the float range through one
    persistent step and through the graph path: the same NaN positions, the
    same bits elsewhere, the same greedy token (a NaN first logit gives 0)."""
    cfg = model.small_config(layers=2)
    w = model.synthetic(cfg, seed=3)
    frames = 6
    prefix = np.random.default_rng(17).standard_normal((frames, cfg.width)).astype(np.float32)
    row = np.random.default_rng(19).standard_normal((1, cfg.width)).astype(np.float32)
    if bad == "nan":
        row[0, 37] = np.nan
    elif bad == "inf":
        row[0, 100] = np.inf
    else:
        row[0, :64] = 3.0e38
    fast = _decoder(backend, w, True, 256)
    slow = _decoder(backend, w, False, 256)
    try:
        assert fast.persistent and not slow.persistent
        fast.decode(prefix, frames)
        slow.decode(prefix, frames)
        lf = fast.decode(row, 1)
        ls = slow.decode(row, 1)
        nf, ns = np.isnan(lf), np.isnan(ls)
        assert np.array_equal(nf, ns)
        assert np.array_equal(lf[~nf].view(np.uint32), ls[~ns].view(np.uint32))
        assert fast.greedy() == slow.greedy() == oracle_lib.greedy(ls)
        kf, vf = fast.kv_read(cfg.layers - 1, frames + 1)
        ks, vs = slow.kv_read(cfg.layers - 1, frames + 1)
        assert np.array_equal(np.isnan(kf), np.isnan(ks)) and np.array_equal(np.isnan(vf), np.isnan(vs))
    finally:
        fast.close()
        slow.close()

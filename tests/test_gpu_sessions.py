"""Lock-step sessions (fah_decoder_generate_sessions): several decoder
sessions over one weight set step together, each weight read once per step.
Every session's tokens and K/V rows must equal those of the same session
decoded alone, and the oracle's."""
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


def _prefixes(cfg, lengths, seed0):
    return [np.random.default_rng(seed0 + i).standard_normal((n, cfg.width)).astype(np.float32)
            for i, n in enumerate(lengths)]


def _alone(backend, w, prefix, steps, capacity):
    """Tokens and K/V rows of one session decoded by itself."""
    from funasrnet_amd.hip import HipDecoder
    d = HipDecoder(backend, w, capacity=capacity)
    try:
        d.decode(prefix, prefix.shape[0])
        toks = d.generate(steps)
        kv = [d.kv_read(layer, prefix.shape[0] + steps) for layer in (0, w.config.layers - 1)]
        return toks, kv
    finally:
        d.close()


@pytest.mark.parametrize("wide", [256, 512], ids=["one_launch", "kernel_per_projection"])
def test_sessions_match_each_session_alone(backend, oracle_lib, wide):
    """Five sessions of the reduced shape, one of capacity `wide`: the batch's
    position bound is the largest capacity, so 256 runs the layers in one
    launch and 512 (past the one-launch step's 320 positions) on the kernel
    per projection. Tokens and K/V rows equal each session decoded alone, and
    the tokens equal the oracle's."""
    from funasrnet_amd.hip import HipDecoder
    cfg = model.small_config(layers=2)
    w = model.synthetic(cfg, seed=21)
    lengths, steps = [9, 17, 30, 1, 64], 12
    prefixes = _prefixes(cfg, lengths, 40)
    parent = HipDecoder(backend, w, capacity=128)
    # The parent takes part too; one session has a different capacity.
    sessions = [parent] + [parent.session(128 if i != 2 else wide) for i in range(1, len(lengths))]
    try:
        for d, p in zip(sessions, prefixes):
            d.decode(p, p.shape[0])
        print(f"sessions small count={len(sessions)} steps={steps} wide={wide}", flush=True)
        toks = HipDecoder.generate_sessions(sessions, steps)
        assert toks.shape == (len(sessions), steps)
        for i, (d, p) in enumerate(zip(sessions, prefixes)):
            assert d.position == p.shape[0] + steps
            alone, kv = _alone(backend, w, p, steps, 128)
            assert toks[i].tolist() == alone.tolist(), i
            for layer, (k, v) in zip((0, cfg.layers - 1), kv):
                ks, vs = d.kv_read(layer, p.shape[0] + steps)
                assert np.array_equal(ks.view(np.uint16), k.view(np.uint16)), (i, layer)
                assert np.array_equal(vs.view(np.uint16), v.view(np.uint16)), (i, layer)
            ref = oracle_lib.Decoder(w, capacity=128)
            try:
                lr = ref.decode(p, p.shape[0])
                expected = []
                for _ in range(steps):
                    t = oracle_lib.greedy(lr)
                    expected.append(t)
                    lr = ref.decode(ref.embed([t]), 1)
                assert toks[i].tolist() == expected, i
            finally:
                ref.close()
        # Sessions continue on their own after a lock-step run.
        more = sessions[1].generate(4)
        ref_d = HipDecoder(backend, w, capacity=128)
        try:
            ref_d.decode(prefixes[1], lengths[1])
            assert ref_d.generate(steps + 4)[steps:].tolist() == more.tolist()
        finally:
            ref_d.close()
    finally:
        for d in sessions[1:]:
            d.close()
        parent.close()


def test_sessions_failed_step_recovers(backend):
    """A one-launch lock-step call stopped by the host
    (fah_decoder_fail_next_step on one session: the batch's error word is set
    before the launch, so every workgroup ends at its entry check) fails with
    the device error, leaves every session at its starting position without
    logits, and the sessions then continue exactly as decoders that never
    failed (FunAsr.cs:167-178 after a Decode of the last token)."""
    from funasrnet_amd import hip
    from funasrnet_amd.hip import HipDecoder
    cfg = model.small_config(layers=2)
    w = model.synthetic(cfg, seed=23)
    lengths = [7, 12, 20]
    prefixes = _prefixes(cfg, lengths, 60)
    parent = HipDecoder(backend, w, capacity=96)
    sessions = [parent] + [parent.session(96) for _ in range(len(lengths) - 1)]
    lib = hip.load()
    try:
        assert all(d.persistent for d in sessions)
        for d, p in zip(sessions, prefixes):
            d.decode(p, p.shape[0])
        print("sessions failure recovery", flush=True)
        first = HipDecoder.generate_sessions(sessions, 3)
        assert lib.fah_decoder_fail_next_step(sessions[1].handle) == hip.OK
        with pytest.raises(RuntimeError, match="stopped by the host"):
            HipDecoder.generate_sessions(sessions, 2)
        for d, p in zip(sessions, prefixes):
            assert d.position == p.shape[0] + 3
        with pytest.raises(RuntimeError, match="no logits"):
            HipDecoder.generate_sessions(sessions, 1)
        for d, t in zip(sessions, first[:, -1]):
            d.decode(d.embed([int(t)]), 1)
        second = HipDecoder.generate_sessions(sessions, 4)
        for i, p in enumerate(prefixes):
            ref = HipDecoder(backend, w, capacity=96)
            try:
                ref.decode(p, p.shape[0])
                a = ref.generate(3).tolist()
                assert a == first[i].tolist(), i
                ref.decode(ref.embed([a[-1]]), 1)
                assert ref.generate(4).tolist() == second[i].tolist(), i
            finally:
                ref.close()
    finally:
        for d in sessions[1:]:
            d.close()
        parent.close()


def test_sessions_reject_bad_batches(backend):
    from funasrnet_amd.hip import HipDecoder
    cfg = model.small_config(layers=1)
    w = model.synthetic(cfg, seed=3)
    a = HipDecoder(backend, w, capacity=32)
    b = a.session()
    other = HipDecoder(backend, w, capacity=32)
    try:
        x = np.random.default_rng(1).standard_normal((4, cfg.width)).astype(np.float32)
        a.decode(x, 4)
        with pytest.raises(RuntimeError, match="no logits"):
            HipDecoder.generate_sessions([a, b], 2)
        b.decode(x, 4)
        other.decode(x, 4)
        with pytest.raises(ValueError, match="share one decoder"):
            HipDecoder.generate_sessions([a, other], 2)
        with pytest.raises(ValueError, match="twice"):
            HipDecoder.generate_sessions([a, b, a], 2)
        with pytest.raises(ValueError, match="exhausted"):
            HipDecoder.generate_sessions([a, b], 29)
        assert a.position == b.position == 4
        t = HipDecoder.generate_sessions([b, a], 3)
        assert t[0].tolist() == t[1].tolist()  # same prefix, same weights
    finally:
        b.close()
        a.close()
        other.close()


def test_sixteen_qwen3_sessions(backend, oracle_lib):
    """Sixteen 150-row N(0,1) prefixes (seeds 1-16) on the full-size model,
    32 lock-step steps: each session's tokens equal its decode alone (three
    checked) and all sixteen equal the oracle's tokens."""
    from funasrnet_amd.hip import HipDecoder
    cfg = model.QWEN3_0_6B
    w = model.synthetic(cfg, seed=0)
    steps, capacity = 32, 192
    prefixes = [np.random.default_rng(seed).standard_normal((150, cfg.width)).astype(np.float32)
                for seed in range(1, 17)]
    parent = HipDecoder(backend, w, capacity=capacity)
    sessions = [parent] + [parent.session() for _ in range(15)]
    try:
        for d, p in zip(sessions, prefixes):
            d.decode(p, 150)
        print("sessions qwen3 count=16 steps=32", flush=True)
        toks = HipDecoder.generate_sessions(sessions, steps)
        for i in (0, 5, 15):
            alone, _ = _alone(backend, w, prefixes[i], steps, capacity)
            assert toks[i].tolist() == alone.tolist(), i
        diverged = []
        for i in range(16):
            ref = oracle_lib.Decoder(w, capacity=capacity)
            try:
                lr = ref.decode(prefixes[i], 150)
                expected = []
                for _ in range(steps):
                    t = oracle_lib.greedy(lr)
                    expected.append(t)
                    lr = ref.decode(ref.embed([t]), 1)
                if toks[i].tolist() != expected:
                    diverged.append(i)
            finally:
                ref.close()
        assert not diverged, f"sessions differing from the oracle: {diverged}"
    finally:
        for d in sessions[1:]:
            d.close()
        parent.close()


def _oracle_tokens(oracle_lib, w, prefix, steps, capacity):
    """Greedy tokens of one session decoded by the oracle: prefix, then
    Greedy -> Embed -> Decode(1) (FunAsr.cs:167-178)."""
    ref = oracle_lib.Decoder(w, capacity=capacity)
    try:
        lr = ref.decode(prefix, prefix.shape[0])
        out = []
        for _ in range(steps):
            t = oracle_lib.greedy(lr)
            out.append(t)
            lr = ref.decode(ref.embed([t]), 1)
        return out
    finally:
        ref.close()


def _run_workers(count, worker):
    import threading
    errors = [None] * count

    def wrapped(i):
        try:
            worker(i)
        except Exception as e:  # reported by the caller
            errors[i] = e

    threads = [threading.Thread(target=wrapped, args=(i,)) for i in range(count)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=300)
    assert not any(t.is_alive() for t in threads)
    return errors


@pytest.mark.parametrize("shape", ["small", "qwen3"])
def test_step_batcher_threads(backend, oracle_lib, shape):
    """Eight worker threads (BoundedInferencePool.cs:78 over the contexts of
    SpeechRuntime.cs:16-23), each decoding its own session (own prefix) with
    the cross-context step batcher, one blocking step per token: every
    session's tokens equal the oracle's decode of that session alone, and the
    steps really ran in batches."""
    from funasrnet_amd.hip import HipDecoder, HipStepBatcher
    cfg = model.small_config(layers=2) if shape == "small" else model.QWEN3_0_6B
    w = model.synthetic(cfg, seed=41)
    count, steps, frames = 8, 24, 20 if shape == "small" else 150
    capacity = frames + steps + 8
    prefixes = [np.random.default_rng(100 + i).standard_normal((frames, cfg.width)).astype(np.float32)
                for i in range(count)]
    expected = [_oracle_tokens(oracle_lib, w, p, steps, capacity) for p in prefixes]
    parent = HipDecoder(backend, w, capacity=capacity)
    sessions = [parent] + [parent.session() for _ in range(count - 1)]
    batcher = HipStepBatcher(parent, max_positions=capacity, window_us=2000)
    results = [None] * count

    def worker(i):
        d = sessions[i]
        d.decode(prefixes[i], frames)
        batcher.join(d)
        results[i] = [batcher.step(d) for _ in range(steps)]
        batcher.leave(d)

    print(f"step batcher {shape}: {count} threads x {steps} steps", flush=True)
    try:
        errors = _run_workers(count, worker)
        assert not any(errors), errors
        diverged = [i for i in range(count) if results[i] != expected[i]]
        assert not diverged, f"sessions differing from the oracle: {diverged}"
        batches, rows = batcher.stats()
        assert rows == count * steps
        assert batches < rows, (batches, rows)  # steps were merged
        print(f"batches {batches}, rows {rows}, mean batch {rows / batches:.2f}", flush=True)
    finally:
        batcher.close()
        for d in sessions[1:]:
            d.close()
        parent.close()


def test_step_batcher_isolates_failures(backend, oracle_lib):
    """One of eight sessions runs out of room (its own capacity, then the
    batcher's bound for another): each gets its error alone, at the step
    where the reference's decoder would throw (QwenDecoder.cs:163), and the
    other sessions' tokens still equal the oracle's."""
    from funasrnet_amd.hip import HipDecoder, HipStepBatcher
    cfg = model.small_config(layers=2)
    w = model.synthetic(cfg, seed=43)
    count, steps, frames = 8, 16, 20
    bound = frames + steps + 4
    prefixes = [np.random.default_rng(300 + i).standard_normal((frames, cfg.width)).astype(np.float32)
                for i in range(count)]
    expected = [_oracle_tokens(oracle_lib, w, p, steps, bound) for p in prefixes]
    parent = HipDecoder(backend, w, capacity=bound)
    # Session 3 holds frames + 6 positions: its 7th step is refused. Session
    # 5 holds more than the batcher's bound; it starts past the bound.
    caps = [bound] * count
    caps[3] = frames + 6
    caps[5] = bound + 64
    sessions = [parent] + [parent.session(caps[i]) for i in range(1, count)]
    batcher = HipStepBatcher(parent, max_positions=bound, window_us=2000)
    results = [[] for _ in range(count)]

    def worker(i):
        d = sessions[i]
        if i == 5:
            d.decode(np.zeros((bound, cfg.width), np.float32), bound)
        else:
            d.decode(prefixes[i], frames)
        batcher.join(d)
        try:
            for _ in range(steps):
                results[i].append(batcher.step(d))
        finally:
            batcher.leave(d)

    print("step batcher failure isolation: 8 threads, sessions 3 and 5 run out of room", flush=True)
    try:
        errors = _run_workers(count, worker)
        assert isinstance(errors[3], ValueError) and "exhausted" in str(errors[3]), errors[3]
        assert results[3] == expected[3][:6]
        assert sessions[3].position == frames + 6
        assert isinstance(errors[5], ValueError) and "bound" in str(errors[5]), errors[5]
        assert results[5] == [] and sessions[5].position == bound
        for i in range(count):
            if i in (3, 5):
                continue
            assert errors[i] is None, (i, errors[i])
            assert results[i] == expected[i], i
        batches, rows = batcher.stats()
        assert rows == (count - 2) * steps + 6
    finally:
        batcher.close()
        for d in sessions[1:]:
            d.close()
        parent.close()


def test_step_batcher_idle_joined_session(backend):
    """A joined session that stops stepping (its worker encodes or prefills)
    holds up the collector once, for one window, not at every step."""
    import time
    from funasrnet_amd.hip import HipDecoder, HipStepBatcher
    cfg = model.small_config(layers=1)
    w = model.synthetic(cfg, seed=45)
    steps, frames, window_us = 20, 8, 100_000
    parent = HipDecoder(backend, w, capacity=64)
    sessions = [parent] + [parent.session() for _ in range(3)]
    batcher = HipStepBatcher(parent, max_positions=64, window_us=window_us)
    x = np.random.default_rng(7).standard_normal((frames, cfg.width)).astype(np.float32)
    try:
        for d in sessions:
            d.decode(x, frames)
            batcher.join(d)
        idle = sessions[3]  # joined, never steps
        results = [None] * 3

        def worker(i):
            results[i] = [batcher.step(sessions[i]) for _ in range(steps)]

        print("step batcher: 3 stepping sessions and 1 idle joined session", flush=True)
        t0 = time.perf_counter()
        errors = _run_workers(3, worker)
        elapsed = time.perf_counter() - t0
        assert not any(errors), errors
        assert results[0] == results[1] == results[2]  # same prefix, same weights
        # Waiting a window at each of the 20 steps would take 2 s.
        assert elapsed < 6 * window_us * 1e-6, elapsed
        batches, rows = batcher.stats()
        assert rows == 3 * steps
        assert idle.position == frames
        for d in sessions:
            batcher.leave(d)
    finally:
        batcher.close()
        for d in sessions[1:]:
            d.close()
        parent.close()

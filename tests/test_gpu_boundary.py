"""The C-ABI contract around the device work: lifetime after
fah_context_destroy (the reference throws ObjectDisposedException,
VulkanQuantizedBackend.cs:54-56), recovery of the persistent step after a
failed launch (forced from the host, every kernel exits normally), and
contexts used from several threads at once (FunAsr.cs:45-47: many FunAsr
instances may share a backend; here each thread has its own context)."""
import ctypes
import os
import threading

import numpy as np
import pytest

from funasrnet_amd import model

pytestmark = pytest.mark.gpu


def _tokens_from_oracle(oracle_lib, ref, logits, steps):
    out = []
    for _ in range(steps):
        t = oracle_lib.greedy(logits)
        out.append(t)
        logits = ref.decode(ref.embed([t]), 1)
    return out, logits


def test_destroy_context_before_its_weight_and_decoder():
    from funasrnet_amd import hip
    lib = hip.load()
    cfg = model.small_config(layers=1)
    w = model.synthetic(cfg, seed=21)
    backend = hip.HipBackend(0)
    weight = hip.HipWeight(backend, w.layers[0].wq)
    decoder = hip.HipDecoder(backend, w, capacity=32)
    x = np.random.default_rng(1).standard_normal((3, cfg.width)).astype(np.float32)
    decoder.decode(x, 3)
    handle = backend.handle
    backend.handle = None  # the Python object must not destroy it again
    assert lib.fah_context_destroy(handle) == hip.OK
    # Calls after destroy report "disposed"; nothing reads freed memory.
    logits = np.empty(cfg.vocab, dtype=np.float32)
    rc = lib.fah_decoder_decode(decoder.handle, x[:1].ctypes.data_as(ctypes.POINTER(ctypes.c_float)), 1,
                                logits.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    assert rc == hip.ERROR_DISPOSED, lib.fah_last_error()
    tok = ctypes.c_int32()
    assert lib.fah_decoder_greedy(decoder.handle, ctypes.byref(tok)) == hip.ERROR_DISPOSED
    assert lib.fah_decoder_set_position(decoder.handle, 0) == hip.ERROR_DISPOSED
    with pytest.raises(RuntimeError, match="disposed"):
        decoder.generate(2)
    # Releasing in either order after the context is gone is fine.
    assert lib.fah_decoder_destroy(decoder.handle) == hip.OK
    decoder.handle = None
    assert lib.fah_weight_release(weight.handle) == hip.OK
    weight.handle = None


def test_sessions_outlive_their_context():
    from funasrnet_amd import hip
    lib = hip.load()
    cfg = model.small_config(layers=1)
    w = model.synthetic(cfg, seed=22)
    backend = hip.HipBackend(0)
    parent = hip.HipDecoder(backend, w, capacity=32)
    child = parent.session()
    handle = backend.handle
    backend.handle = None
    assert lib.fah_context_destroy(handle) == hip.OK
    # The parent goes first; the session still holds the weights and state.
    assert lib.fah_decoder_destroy(parent.handle) == hip.OK
    parent.handle = None
    assert lib.fah_decoder_set_position(child.handle, 0) == hip.ERROR_DISPOSED
    assert lib.fah_decoder_destroy(child.handle) == hip.OK
    child.handle = None


@pytest.mark.parametrize("shape", ["small", "qwen3"])
def test_recovery_after_a_failed_persistent_step(oracle_lib, shape):
    """The host presets the error word: the next generate ends at the kernel's
    entry check and reports an error without advancing; the state is restored
    (epoch, device position), so a new decode of the same row and the tokens
    after it match the oracle, with host and device positions equal."""
    from funasrnet_amd import hip
    cfg = model.small_config(layers=2) if shape == "small" else model.QWEN3_0_6B
    w = model.synthetic(cfg, seed=23)
    frames = 12 if shape == "small" else 150
    prefix = np.random.default_rng(24).standard_normal((frames, cfg.width)).astype(np.float32)
    backend = hip.HipBackend(0)
    gpu = hip.HipDecoder(backend, w, capacity=256)
    ref = oracle_lib.Decoder(w, capacity=256)
    lib = hip.load()
    try:
        assert gpu.persistent
        print(f"failure recovery {shape}", flush=True)
        gpu.decode(prefix, frames)
        lr = ref.decode(prefix, frames)
        toks = gpu.generate(4).tolist()
        expected, lr = _tokens_from_oracle(oracle_lib, ref, lr, 4)
        assert toks == expected
        assert gpu.position == ref.position == frames + 4
        # The failed call: every workgroup ends at its entry check.
        assert lib.fah_decoder_fail_next_step(gpu.handle) == hip.OK
        with pytest.raises(RuntimeError, match="stopped by the host"):
            gpu.generate(3)
        assert gpu.position == frames + 4
        with pytest.raises(RuntimeError, match="no logits"):
            gpu.greedy()
        # The same failure in a decode of a host row.
        x = gpu.embed([expected[-1]])
        assert lib.fah_decoder_fail_next_step(gpu.handle) == hip.OK
        with pytest.raises(RuntimeError, match="stopped by the host"):
            gpu.decode(x, 1)
        assert gpu.position == frames + 4
        # Recovered: the oracle continues from the same row.
        lg = gpu.decode(x, 1)
        lr = ref.decode(ref.embed([expected[-1]]), 1)
        assert np.abs(lg.astype(np.float64) - lr).max() <= 1e-2
        assert gpu.greedy() == oracle_lib.greedy(lr)
        toks = gpu.generate(6).tolist()
        expected, lr = _tokens_from_oracle(oracle_lib, ref, lr, 6)
        assert toks == expected
        assert gpu.position == ref.position == frames + 11
        # The K/V row of every decoded position sits where the oracle has it.
        kg, vg = gpu.kv_read(cfg.layers - 1, frames + 11)
        kr, vr = ref.kv(cfg.layers - 1)
        assert np.abs(kg.astype(np.float32) - kr.reshape(kg.shape)).max() < 1e-2
        assert np.abs(vg.astype(np.float32) - vr.reshape(vg.shape)).max() < 1e-2
    finally:
        gpu.close()
        ref.close()
        backend.close()


def test_fail_hook_declined_on_the_graph_path():
    from funasrnet_amd import hip
    cfg = model.small_config(layers=1)
    w = model.synthetic(cfg, seed=25)
    old = os.environ.get("FAH_PERSISTENT")
    os.environ["FAH_PERSISTENT"] = "0"
    backend = hip.HipBackend(0)
    try:
        gpu = hip.HipDecoder(backend, w, capacity=32)
    finally:
        if old is None:
            del os.environ["FAH_PERSISTENT"]
        else:
            os.environ["FAH_PERSISTENT"] = old
    try:
        assert hip.load().fah_decoder_fail_next_step(gpu.handle) == hip.DECLINED
    finally:
        gpu.close()
        backend.close()


def test_two_contexts_on_two_threads():
    """Two contexts, each with its own Qwen3-0.6B decoder, generate 32 tokens
    each from two threads at once (every persistent step keeps the device to
    itself): the tokens equal a single-context run, and no step times out."""
    from funasrnet_amd import hip
    cfg = model.QWEN3_0_6B
    w = model.synthetic(cfg, seed=0)
    prefixes = [np.random.default_rng(s).standard_normal((150, cfg.width)).astype(np.float32) for s in (31, 32)]
    steps = 32
    alone = []
    backend = hip.HipBackend(0)
    try:
        d = hip.HipDecoder(backend, w, capacity=256)
        try:
            for p in prefixes:
                d.set_position(0)
                d.decode(p, 150)
                alone.append(d.generate(steps).tolist())
        finally:
            d.close()
    finally:
        backend.close()
    print("two contexts, two threads", flush=True)
    backends = [hip.HipBackend(0), hip.HipBackend(0)]
    decoders = [hip.HipDecoder(b, w, capacity=256) for b in backends]
    results, errors = [None, None], []

    def run(i):
        try:
            decoders[i].decode(prefixes[i], 150)
            got = []
            for _ in range(4):  # several calls, so the threads interleave
                got.extend(decoders[i].generate(steps // 4).tolist())
            results[i] = got
        except Exception as e:  # reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    try:
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=300)
        assert not any(t.is_alive() for t in threads)
        assert not errors, errors
        assert results == alone
        assert all(hip.load().fah_decoder_persistent(d.handle) == 2 for d in decoders)
    finally:
        for d in decoders:
            d.close()
        for b in backends:
            b.close()

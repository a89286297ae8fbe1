"""Prefill (QwenDecoder.Decode with many rows at once) on the Q8_0 GEMMs
(the few-frame kernel up to 16 rows, MFMA above) against the row-by-row
decode path and the oracle: identical logits bits and F16 KV rows, then
identical greedy tokens when decoding continues."""
import os

import numpy as np
import pytest

from funasrnet_amd import model

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-2, 1e-3


@pytest.fixture(scope="module")
def backend():
    from funasrnet_amd.hip import HipBackend
    b = HipBackend(0)
    yield b
    b.close()


def _decode(decoder, x, row_by_row):
    old = os.environ.get("FAH_PREFILL")
    os.environ["FAH_PREFILL"] = "0" if row_by_row else "1"
    try:
        return decoder.decode(x, x.shape[0])
    finally:
        if old is None:
            del os.environ["FAH_PREFILL"]
        else:
            os.environ["FAH_PREFILL"] = old


@pytest.mark.parametrize("shape,frames", [("small", 5), ("small", 16), ("small", 37), ("small", 130),
                                          ("qwen3", 12), ("qwen3", 150), ("qwen3", 375), ("qwen3", 750)])
def test_prefill_matches_row_by_row(backend, oracle_lib, shape, frames):
    """Every size, including the long audio prefixes of 375 and 750 rows:
    the batched prefill equals the row-by-row decode bit for bit (logits and
    every layer's K/V rows), and matches the oracle (logits within the
    tolerance and bit-identical, the greedy token, then 8 generated tokens)."""
    from funasrnet_amd.hip import HipDecoder
    cfg = model.small_config(layers=2) if shape == "small" else model.QWEN3_0_6B
    w = model.synthetic(cfg, seed=5)
    prefix = np.random.default_rng(frames).standard_normal((frames, cfg.width)).astype(np.float32)
    capacity = frames + 64
    batched = HipDecoder(backend, w, capacity=capacity)
    rows = HipDecoder(backend, w, capacity=capacity)
    try:
        print(f"prefill {shape} frames={frames}", flush=True)
        lb = _decode(batched, prefix, row_by_row=False)
        lr = _decode(rows, prefix, row_by_row=True)
        assert np.array_equal(lb.view(np.uint32), lr.view(np.uint32))
        assert batched.position == rows.position == frames
        for layer in range(cfg.layers):
            kb, vb = batched.kv_read(layer, frames)
            kr, vr = rows.kv_read(layer, frames)
            assert np.array_equal(kb, kr) and np.array_equal(vb, vr), layer
        tb = batched.generate(8)
        tr = rows.generate(8)
        assert np.array_equal(tb, tr)
        ref = oracle_lib.Decoder(w, capacity=capacity)
        try:
            lo = ref.decode(prefix, frames)
            diff = np.abs(lb.astype(np.float64) - lo.astype(np.float64))
            assert diff.max() <= ATOL
            assert np.all(diff <= RTOL * np.maximum(1.0, np.abs(lo)))
            assert np.array_equal(lb.view(np.uint32), lo.view(np.uint32))
            assert int(np.argmax(lo)) == int(tb[0]) == oracle_lib.greedy(lo)
            for layer in (0, cfg.layers - 1):
                kb, vb = batched.kv_read(layer, frames)
                ko, vo = ref.kv(layer)
                assert np.array_equal(kb.astype(np.float32), ko.reshape(kb.shape)), layer
                assert np.array_equal(vb.astype(np.float32), vo.reshape(vb.shape)), layer
            expected = []
            for _ in range(8):
                t = oracle_lib.greedy(lo)
                expected.append(t)
                lo = ref.decode(ref.embed([t]), 1)
            assert tb.tolist() == expected
        finally:
            ref.close()
    finally:
        batched.close()
        rows.close()


def test_prefill_in_two_calls_matches_one(backend):
    """A prefix given in two parts continues from the cached K/V rows."""
    from funasrnet_amd.hip import HipDecoder
    cfg = model.small_config(layers=2)
    w = model.synthetic(cfg, seed=9)
    prefix = np.random.default_rng(3).standard_normal((90, cfg.width)).astype(np.float32)
    one = HipDecoder(backend, w, capacity=128)
    two = HipDecoder(backend, w, capacity=128)
    try:
        l1 = _decode(one, prefix, row_by_row=False)
        two.decode(prefix[:41], 41)
        l2 = _decode(two, prefix[41:], row_by_row=False)
        assert np.array_equal(l1.view(np.uint32), l2.view(np.uint32))
    finally:
        one.close()
        two.close()

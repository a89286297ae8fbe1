"""The oracle's decoder (oracle_decoder_*, a composition of the pinned
functions) against properties the reference's code fixes:

* Decode of many rows at once equals the same rows decoded one at a time
  (the grouped projections keep the single-frame float order,
  TensorMath.QuantizedGroupAvx.cs:17-199; attention is causal,
  QwenDecoder.cs:206-224): identical logits and K/V bits.
* RestorePrefix (QwenDecoder.cs:122-137): rewinding the position and decoding
  the same rows again gives the same logits.
* Capacity (QwenDecoder.cs:163-166): decoding past it is rejected before any
  state changes.
* Embed (QwenDecoder.cs:143-152, Gguf.cs:326-345) is q * scale of the row.
"""
import numpy as np
import pytest

from funasrnet_amd import model


@pytest.fixture(scope="module")
def weights():
    return model.synthetic(model.small_config(layers=2, vocab=512), seed=31)


def _rows(cfg, n, seed):
    return np.random.default_rng(seed).standard_normal((n, cfg.width)).astype(np.float32)


def test_batched_rows_equal_rows_one_at_a_time(oracle_lib, weights):
    cfg = weights.config
    x = _rows(cfg, 11, 1)
    batched = oracle_lib.Decoder(weights, capacity=32)
    single = oracle_lib.Decoder(weights, capacity=32)
    try:
        lb = batched.decode(x, 11)
        for t in range(11):
            ls = single.decode(x[t:t + 1], 1)
        assert np.array_equal(lb.view(np.uint32), ls.view(np.uint32))
        for layer in range(cfg.layers):
            kb, vb = batched.kv(layer)
            ks, vs = single.kv(layer)
            assert np.array_equal(kb.view(np.uint32), ks.view(np.uint32))
            assert np.array_equal(vb.view(np.uint32), vs.view(np.uint32))
        # The cached rows hold F16 values (QwenDecoder.cs:195-203).
        k, _ = batched.kv(0)
        assert np.array_equal(k, k.astype(np.float16).astype(np.float32))
    finally:
        batched.close()
        single.close()


def test_rows_split_over_calls_equal_one_call(oracle_lib, weights):
    cfg = weights.config
    x = _rows(cfg, 9, 2)
    one = oracle_lib.Decoder(weights, capacity=16)
    two = oracle_lib.Decoder(weights, capacity=16)
    try:
        l1 = one.decode(x, 9)
        two.decode(x[:4], 4, output_logits=False)
        l2 = two.decode(x[4:], 5)
        assert np.array_equal(l1.view(np.uint32), l2.view(np.uint32))
        assert one.position == two.position == 9
    finally:
        one.close()
        two.close()


def test_restore_prefix_replays_identically(oracle_lib, weights):
    cfg = weights.config
    prefix, tail = _rows(cfg, 6, 3), _rows(cfg, 3, 4)
    d = oracle_lib.Decoder(weights, capacity=16)
    try:
        d.decode(prefix, 6, output_logits=False)
        first = d.decode(tail, 3)
        d.set_position(6)
        again = d.decode(tail, 3)
        assert np.array_equal(first.view(np.uint32), again.view(np.uint32))
        d.reset()
        assert d.position == 0
    finally:
        d.close()


def test_capacity_is_enforced_before_state_changes(oracle_lib, weights):
    cfg = weights.config
    d = oracle_lib.Decoder(weights, capacity=4)
    try:
        d.decode(_rows(cfg, 3, 5), 3, output_logits=False)
        with pytest.raises(Exception, match="exhausted"):
            d.decode(_rows(cfg, 2, 6), 2)
        assert d.position == 3
        with pytest.raises(Exception):
            d.set_position(5)
    finally:
        d.close()


def test_embed_is_q_times_scale(oracle_lib, weights):
    cfg = weights.config
    d = oracle_lib.Decoder(weights, capacity=4)
    try:
        tokens = [0, 5, cfg.vocab - 1]
        rows = d.embed(tokens)
        e = weights.token_embd
        for i, t in enumerate(tokens):
            expected = e.quantized[t].astype(np.float32) * np.repeat(e.scales[t], 32)
            assert np.array_equal(rows[i], expected.astype(np.float32))
        with pytest.raises(Exception):
            d.embed([cfg.vocab])
    finally:
        d.close()


def test_greedy_token_is_first_maximum(oracle_lib, weights):
    cfg = weights.config
    d = oracle_lib.Decoder(weights, capacity=4)
    try:
        logits = d.decode(_rows(cfg, 2, 7), 2)
        assert oracle_lib.greedy(logits) == int(np.argmax(logits))
    finally:
        d.close()

"""GPU parity of the device-resident decoder (QwenDecoder.Decode) against the
oracle: logits within the north-star tolerance (max-abs 1e-2, relative 1e-3)
and, since every step follows the oracle's float order, bit-identical; F16
KV cache rows and greedy tokens identical."""
import numpy as np
import pytest

from funasrnet_amd import model

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-2, 1e-3


def assert_logits_close(got, expected):
    diff = np.abs(got.astype(np.float64) - expected.astype(np.float64))
    assert np.all(np.isfinite(got))
    assert diff.max() <= ATOL, diff.max()
    assert np.all(diff <= RTOL * np.maximum(1.0, np.abs(expected))), (diff / np.maximum(1.0, np.abs(expected))).max()


@pytest.fixture(scope="module")
def backend():
    from funasrnet_amd.hip import HipBackend
    b = HipBackend(0)
    yield b
    b.close()


def _run_pair(backend, oracle_lib, weights, prefix, steps, capacity=512):
    from funasrnet_amd.hip import HipDecoder
    gpu = HipDecoder(backend, weights, capacity=capacity)
    ref = oracle_lib.Decoder(weights, capacity=capacity)
    try:
        lg = gpu.decode(prefix, prefix.shape[0])
        lr = ref.decode(prefix, prefix.shape[0])
        assert_logits_close(lg, lr)
        exact = [np.array_equal(lg.view(np.uint32), lr.view(np.uint32))]
        tokens_gpu, tokens_ref = [gpu.greedy()], [oracle_lib.greedy(lr)]
        assert tokens_gpu[0] == tokens_ref[0] == int(np.argmax(lr))
        for _ in range(steps):
            lg = gpu.decode(gpu.embed([tokens_gpu[-1]]), 1)
            lr = ref.decode(ref.embed([tokens_ref[-1]]), 1)
            assert_logits_close(lg, lr)
            exact.append(np.array_equal(lg.view(np.uint32), lr.view(np.uint32)))
            tokens_gpu.append(gpu.greedy())
            tokens_ref.append(oracle_lib.greedy(lr))
        assert tokens_gpu == tokens_ref
        pos = gpu.position
        assert pos == ref.position == prefix.shape[0] + steps
        for layer in (0, weights.config.layers - 1):
            kg, vg = gpu.kv_read(layer, pos)
            kr, vr = ref.kv(layer)
            assert np.array_equal(kg.astype(np.float32), kr.reshape(kg.shape).astype(np.float32)), layer
            assert np.array_equal(vg.astype(np.float32), vr.reshape(vg.shape).astype(np.float32)), layer
        assert all(exact), f"bit-exact logits in {sum(exact)} of {len(exact)} steps"
        return exact
    finally:
        gpu.close()
        ref.close()


def test_small_decoder_matches_oracle(backend, oracle_lib):
    w = model.synthetic(model.small_config(layers=2), seed=3)
    prefix = np.random.default_rng(1).standard_normal((20, w.config.width)).astype(np.float32)
    _run_pair(backend, oracle_lib, w, prefix, steps=12)


def test_qwen3_1_7b_shaped_decoder_matches_oracle(backend, oracle_lib):
    """Qwen3-1.7B's shape (width 2048, 16/8 heads, ffn 6144; two layers and
    a 16,384-token vocabulary to keep the oracle quick): no persistent
    instantiation, so the multi-kernel step runs (the down projection's
    GEMV on 16 register chunks), and the prefix goes row by row (the
    prefill GEMMs take ffn up to 3072). Bit-exact logits, K/V rows and
    tokens against the oracle."""
    cfg = model.DecoderConfig(width=2048, heads=16, kv_heads=8, layers=2, ffn=6144, vocab=16384)
    w = model.synthetic(cfg, seed=17)
    prefix = np.random.default_rng(18).standard_normal((6, cfg.width)).astype(np.float32)
    _run_pair(backend, oracle_lib, w, prefix, steps=6, capacity=64)


@pytest.mark.parametrize("name,width,ffn", [("4b", 2560, 9728), ("8b", 4096, 12288)])
def test_qwen3_grouped_by_four_shapes_match_oracle(backend, oracle_lib, name, width, ffn):
    """Qwen3-4B and 8B shapes (32 query heads on 8 KV heads: four a group,
    the value kernel's 8-channel slices; two layers, a 16,384-token
    vocabulary): bit-exact logits, K/V rows and tokens against the oracle."""
    cfg = model.DecoderConfig(width=width, heads=32, kv_heads=8, layers=2, ffn=ffn, vocab=16384)
    w = model.synthetic(cfg, seed=19)
    prefix = np.random.default_rng(20).standard_normal((5, cfg.width)).astype(np.float32)
    print(f"qwen3 {name} shape", flush=True)
    _run_pair(backend, oracle_lib, w, prefix, steps=4, capacity=64)


def test_grouped_by_four_long_cache_matches_oracle(backend, oracle_lib):
    """The 4B shape after 700 cached F16 N(0,1) rows: the value kernel over
    three 256-position blocks with four heads' denominators (exact block sums
    or the residue chains), bit-exact against the oracle for the first step
    and the next four greedy tokens."""
    from funasrnet_amd.hip import HipDecoder
    cfg = model.DecoderConfig(width=2560, heads=32, kv_heads=8, layers=2, ffn=9728, vocab=16384)
    w = model.synthetic(cfg, seed=21)
    positions, capacity = 700, 768
    rng = np.random.default_rng(22)
    kv = [(rng.standard_normal((positions, cfg.kv_width)).astype(np.float16),
           rng.standard_normal((positions, cfg.kv_width)).astype(np.float16)) for _ in range(cfg.layers)]
    x = rng.standard_normal((1, cfg.width)).astype(np.float32)
    gpu = HipDecoder(backend, w, capacity=capacity)
    ref = oracle_lib.Decoder(w, capacity=capacity)
    try:
        for layer, (k, v) in enumerate(kv):
            gpu.kv_write(layer, k, v)
            ref.set_kv(layer, k.astype(np.float32), v.astype(np.float32))
        gpu.set_position(positions)
        ref.set_position(positions)
        print("qwen3 4b shape, 700 cached positions", flush=True)
        lg = gpu.decode(x, 1)
        lr = ref.decode(x, 1)
        assert np.array_equal(lg.view(np.uint32), lr.view(np.uint32))
        tokens = gpu.generate(4).tolist()
        expected = []
        for _ in range(4):
            t = oracle_lib.greedy(lr)
            expected.append(t)
            lr = ref.decode(ref.embed([t]), 1)
        assert tokens == expected
    finally:
        gpu.close()
        ref.close()


def test_small_decoder_fp32_scales(backend, oracle_lib):
    """Scales that fp16 cannot hold keep an fp32 plane on the device."""
    w = model.synthetic(model.small_config(layers=1), seed=4)
    for L in w.layers:
        for t in (L.wq, L.wk, L.wv, L.wo, L.gate, L.up, L.down):
            t.scales = (t.scales * np.float32(1.0000001)).astype(np.float32)
    w.token_embd.scales = (w.token_embd.scales * np.float32(1.0000001)).astype(np.float32)
    prefix = np.random.default_rng(2).standard_normal((9, w.config.width)).astype(np.float32)
    _run_pair(backend, oracle_lib, w, prefix, steps=4)


def test_generate_matches_host_loop(backend, oracle_lib):
    """fah_decoder_generate (device token feedback) == the Transcribe loop
    (FunAsr.cs:167-178) run on the oracle."""
    from funasrnet_amd.hip import HipDecoder
    w = model.synthetic(model.small_config(layers=2), seed=5)
    prefix = np.random.default_rng(3).standard_normal((16, w.config.width)).astype(np.float32)
    gpu = HipDecoder(backend, w, capacity=256)
    ref = oracle_lib.Decoder(w, capacity=256)
    try:
        gpu.decode(prefix, 16)
        lr = ref.decode(prefix, 16)
        toks = gpu.generate(24)
        expected = []
        for _ in range(24):
            t = oracle_lib.greedy(lr)
            expected.append(t)
            lr = ref.decode(ref.embed([t]), 1)
        assert toks.tolist() == expected
        assert gpu.position == 40
        assert gpu.greedy() == oracle_lib.greedy(lr)
    finally:
        gpu.close()
        ref.close()


def test_capacity_exhaustion_and_restore(backend):
    from funasrnet_amd.hip import HipDecoder
    w = model.synthetic(model.small_config(layers=1), seed=6)
    gpu = HipDecoder(backend, w, capacity=8)
    try:
        x = np.zeros((8, w.config.width), dtype=np.float32)
        gpu.decode(x, 8, output_logits=False)
        with pytest.raises(ValueError):
            gpu.decode(x[:1], 1)
        gpu.set_position(4)  # RestorePrefix
        assert gpu.position == 4
        gpu.decode(x[:4], 4)
        gpu.reset()
        assert gpu.position == 0
    finally:
        gpu.close()


def test_qwen3_0_6b_decode_tokens_match(backend, oracle_lib):
    """Qwen3-0.6B at full size: 150-row N(0,1) prefix, then 128 greedy steps;
    the token sequence must equal the oracle's."""
    from funasrnet_amd.hip import HipDecoder
    w = model.synthetic(model.QWEN3_0_6B, seed=0)
    prefix = np.random.default_rng(0).standard_normal((150, 1024)).astype(np.float32)
    gpu = HipDecoder(backend, w, capacity=2048)
    ref = oracle_lib.Decoder(w, capacity=2048)
    try:
        print("qwen3 150 rows + 128 steps", flush=True)
        lg = gpu.decode(prefix, 150)
        lr = ref.decode(prefix, 150)
        assert_logits_close(lg, lr)
        assert np.array_equal(lg.view(np.uint32), lr.view(np.uint32))
        toks = gpu.generate(128)
        expected = []
        for _ in range(128):
            t = oracle_lib.greedy(lr)
            expected.append(t)
            lr = ref.decode(ref.embed([t]), 1)
        mismatch = [i for i, (a, b) in enumerate(zip(toks.tolist(), expected)) if a != b]
        assert not mismatch, f"first divergence at step {mismatch[0]}"
        # The logits after the 128 steps, and the K/V rows of every position.
        x = gpu.embed([expected[-1]])
        lg = gpu.decode(x, 1)
        lr = ref.decode(ref.embed([expected[-1]]), 1)
        assert_logits_close(lg, lr)
        assert np.array_equal(lg.view(np.uint32), lr.view(np.uint32))
        for layer in (0, 27):
            kg, vg = gpu.kv_read(layer, 279)
            kr, vr = ref.kv(layer)
            assert np.array_equal(kg.astype(np.float32), kr.reshape(kg.shape)), layer
            assert np.array_equal(vg.astype(np.float32), vr.reshape(vg.shape)), layer
    finally:
        gpu.close()
        ref.close()


def test_decoder_from_gguf_blocks(backend, tmp_path):
    """A decoder built from the GGUF file's raw Q8_0 blocks (split on the
    device) decodes exactly like one built from the unpacked planes."""
    from funasrnet_amd import gguf
    from funasrnet_amd.hip import HipDecoder
    cfg = model.small_config(layers=2)
    w = model.synthetic(cfg, seed=17)
    path = str(tmp_path / "small.gguf")
    model.to_gguf(w, path)
    raw = model.from_gguf(gguf.Gguf.read(path, raw_q8=True))
    unpacked = model.from_gguf(gguf.Gguf.read(path))
    assert raw.layers[0].wq.quantized is None and raw.layers[0].wq.blocks is not None
    prefix = np.random.default_rng(18).standard_normal((9, cfg.width)).astype(np.float32)
    a = HipDecoder(backend, raw, capacity=64)
    b = HipDecoder(backend, unpacked, capacity=64)
    try:
        assert a.weight_bytes == b.weight_bytes
        la, lb = a.decode(prefix, 9), b.decode(prefix, 9)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
        assert a.generate(6).tolist() == b.generate(6).tolist()
    finally:
        a.close()
        b.close()

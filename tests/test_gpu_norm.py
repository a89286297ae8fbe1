"""RMSNorm on the GPU against the oracle, bit for bit, on rows where the
GPU's pairwise-tree square sum rounds to another float mean than the
reference's four ordered chains (TensorMath.Elementwise.cs:58-71): the
kernels must notice and take the reference's order there."""
import os

import numpy as np
import pytest

from funasrnet_amd import model
from tests import norm_rows

pytestmark = pytest.mark.gpu
f32 = np.float32


@pytest.fixture(scope="module")
def backend():
    from funasrnet_amd.hip import HipBackend
    b = HipBackend(0, minimum_operations=0)
    yield b
    b.close()


def _rows(oracle_lib, width):
    rng = np.random.default_rng(width)
    rows = [norm_rows.mismatching(oracle_lib, width, 24, seed=width + 1),
            norm_rows.midpoint(width)[None],
            rng.standard_normal((16, width)).astype(f32),
            (rng.standard_normal((8, width)) * np.exp(rng.standard_normal((8, width)) * 4)).astype(f32)]
    special = np.ones((5, width), f32)
    special[0] = 0.0
    special[1, 5] = np.inf
    special[2, 7] = np.nan
    special[3] *= f32(1e-40)  # subnormal values
    special[4, ::3] = f32(-3e18)
    rows.append(special)
    return np.concatenate(rows)


@pytest.mark.parametrize("width", [128, 1024])
def test_rms_norm_device_matches_oracle(backend, oracle_lib, width):
    """fah_rms_norm_device (the decoder's QK-norm arithmetic at width 128,
    its layer-norm arithmetic at 1024) equals oracle_rms_norm on crafted
    rows (tree and reference means differ), a rounding-midpoint row, random
    rows and special values."""
    from funasrnet_amd import device as dev
    x = _rows(oracle_lib, width)
    scale = np.random.default_rng(5).standard_normal(width).astype(f32)
    print(f"rms norm width {width}: {x.shape[0]} rows", flush=True)
    xd, sd = dev.DeviceArray.from_numpy(x), dev.DeviceArray.from_numpy(scale)
    yd = dev.DeviceArray(x.shape, np.float32)
    backend.rms_norm_device(xd.ptr, x.shape[0], width, sd.ptr, 1e-6, yd.ptr)
    backend.synchronize()
    got = yd.numpy()
    expected = oracle_lib.rms_norm(x, width, scale, 1e-6)
    nan = np.isnan(expected)
    assert np.array_equal(np.isnan(got), nan)
    bad = [i for i in range(x.shape[0]) if not np.array_equal(got[i][~nan[i]].view(np.uint32),
                                                               expected[i][~nan[i]].view(np.uint32))]
    assert not bad, f"rows differing from the oracle: {bad}"


def _one_layer():
    cfg = model.DecoderConfig(layers=1, vocab=4096)
    return cfg, model.synthetic(cfg, seed=17)


@pytest.mark.parametrize("path", ["persistent", "graph"])
def test_decode_norm_on_crafted_rows(backend, oracle_lib, path):
    """A one-layer Qwen3-0.6B-shaped decoder fed crafted embedding rows one
    at a time: layer 0's attention norm sees each row as it is, so its raw
    q|k|v projections (whose Q8_0 block scales move with the norm's inverse)
    and the logits must equal the oracle's bit for bit."""
    from funasrnet_amd.hip import HipDecoder
    cfg, w = _one_layer()
    rows = norm_rows.mismatching(oracle_lib, cfg.width, 6, seed=99)
    old = os.environ.get("FAH_PERSISTENT")
    os.environ["FAH_PERSISTENT"] = "1" if path == "persistent" else "0"
    try:
        d = HipDecoder(backend, w, capacity=32)
    finally:
        if old is None:
            del os.environ["FAH_PERSISTENT"]
        else:
            os.environ["FAH_PERSISTENT"] = old
    ref = oracle_lib.Decoder(w, capacity=32)
    L = w.layers[0]
    try:
        assert d.persistent == (path == "persistent")
        print(f"crafted norm rows through the {path} step", flush=True)
        for i, x in enumerate(rows):
            lg = d.decode(x[None], 1)
            lr = ref.decode(x[None], 1)
            h = oracle_lib.rms_norm(x, cfg.width, L.attn_norm, cfg.eps)
            qkv = np.concatenate([oracle_lib.linear(h[None], t.quantized, t.scales) .ravel()
                                  for t in (L.wq, L.wk, L.wv)])
            assert np.array_equal(d.trace("qkv").view(np.uint32), qkv.view(np.uint32)), i
            assert np.array_equal(lg.view(np.uint32), lr.view(np.uint32)), i
    finally:
        d.close()
        ref.close()


def test_prefill_norm_on_crafted_rows(backend, oracle_lib):
    """The same rows as one prefill (norm_quantize_rows_kernel and the
    batched projections): logits and layer 0's K/V rows equal the oracle's."""
    from funasrnet_amd.hip import HipDecoder
    cfg, w = _one_layer()
    rows = norm_rows.mismatching(oracle_lib, cfg.width, 8, seed=7)
    d = HipDecoder(backend, w, capacity=32)
    ref = oracle_lib.Decoder(w, capacity=32)
    try:
        print("crafted norm rows as one prefill", flush=True)
        lg = d.decode(rows, rows.shape[0])
        lr = ref.decode(rows, rows.shape[0])
        assert np.array_equal(lg.view(np.uint32), lr.view(np.uint32))
        k, v = d.kv_read(0, rows.shape[0])
        kr, vr = ref.kv(0)
        assert np.array_equal(k.astype(f32).ravel(), kr)
        assert np.array_equal(v.astype(f32).ravel(), vr)
    finally:
        d.close()
        ref.close()

"""GPU parity of the Q8_0 path through the C ABI: activation quantisation and
int32 block dots bit-exact, projections bit-exact against the oracle."""
import os

import numpy as np
import pytest

from tests.golden.make_golden import q8_kat_case

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")

# Decoder projection shapes (K -> N) of Qwen3-0.6B.
SHAPES = [(1024, 2048), (1024, 1024), (2048, 1024), (1024, 3072), (3072, 1024), (1024, 151936)]


@pytest.fixture(scope="module")
def backend():
    from funasrnet_amd.hip import HipBackend
    b = HipBackend(0, minimum_operations=0)
    yield b
    b.close()


@pytest.fixture(scope="module")
def dev():
    from funasrnet_amd import device
    return device


def _weights(rng, rows, cols):
    from funasrnet_amd.model import Q8Tensor
    q = rng.integers(-127, 128, size=(rows, cols), dtype=np.int8)
    s = (np.abs(rng.standard_normal(rows * cols // 32, dtype=np.float32)) * np.float32(0.02 / 127)).astype(np.float16)
    return Q8Tensor("w", q, s.astype(np.float32).reshape(rows, -1))


def test_quantize_golden_bit_exact(backend, dev):
    g = np.load(os.path.join(GOLDEN, "quantize_kat.npz"))
    n = g["input"].size
    x = dev.DeviceArray.from_numpy(g["input"])
    q = dev.DeviceArray(n, np.int8)
    s = dev.DeviceArray(n // 32, np.float32)
    backend.quantize_device(x.ptr, n, q.ptr, s.ptr)
    backend.synchronize()
    qh, sh = q.numpy(), s.numpy()
    assert np.array_equal(qh, g["q"])
    nan = np.isnan(g["scales"])
    assert np.array_equal(np.isnan(sh), nan)
    assert np.array_equal(sh[~nan].view(np.uint32), g["scales"][~nan].view(np.uint32))


def test_quantize_random_bit_exact(backend, dev, oracle_lib):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(1 << 16), rng.standard_normal(1 << 14) * 10.0 ** rng.integers(-38, 38, 1 << 14)])
    x = x.astype(np.float32)
    xd = dev.DeviceArray.from_numpy(x)
    q = dev.DeviceArray(x.size, np.int8)
    s = dev.DeviceArray(x.size // 32, np.float32)
    backend.quantize_device(xd.ptr, x.size, q.ptr, s.ptr)
    backend.synchronize()
    q0, s0 = oracle_lib.quantize(x)
    assert np.array_equal(q.numpy(), q0)
    assert np.array_equal(s.numpy().view(np.uint32), s0.view(np.uint32))


@pytest.mark.parametrize("cols,rows", SHAPES)
def test_block_dots_bit_exact(backend, dev, oracle_lib, cols, rows):
    rng = np.random.default_rng(cols + rows)
    w = _weights(rng, rows, cols)
    w.quantized[0, :32] = -128  # the kernels must accept -128 weights
    hw = backend.weight(w)
    x = rng.standard_normal(cols).astype(np.float32)
    xq, xs = oracle_lib.quantize(x)
    q = dev.DeviceArray.from_numpy(xq)
    dots = dev.DeviceArray(rows * cols // 32, np.int32)
    backend.block_dots_device(q.ptr, hw, dots.ptr)
    backend.synchronize()
    assert np.array_equal(dots.numpy().reshape(rows, -1), oracle_lib.block_dots(xq, w.quantized))


# Inputs wider than the 0.6B decoder's: Qwen3-1.7B's down projection
# (6144 -> 2048), 8B's width of ffn (12288), the GEMV's limit (16384).
LARGE_K = [(6144, 2048), (12288, 1024), (16384, 64)]


@pytest.mark.parametrize("cols,rows", SHAPES + LARGE_K)
def test_gemv_bit_exact(backend, dev, oracle_lib, cols, rows):
    rng = np.random.default_rng(cols * 7 + rows)
    w = _weights(rng, rows, cols)
    hw = backend.weight(w)
    x = rng.standard_normal(cols).astype(np.float32)
    xq, xs = oracle_lib.quantize(x)
    q, s = dev.DeviceArray.from_numpy(xq), dev.DeviceArray.from_numpy(xs)
    out = dev.DeviceArray(rows, np.float32)
    assert backend.gemv_device(q.ptr, s.ptr, 1, hw, out.ptr) == 0
    backend.synchronize()
    expected = oracle_lib.gemv_quantized(xq, xs, w.quantized, w.scales)[0]
    assert np.array_equal(out.numpy().view(np.uint32), expected.view(np.uint32))


@pytest.mark.parametrize("frames", [1, 3, 17])
@pytest.mark.parametrize("width", [32, 96, 1024])
@pytest.mark.parametrize("rows", [1, 3, 19, 32])
def test_quantized_linear_reference_kat(backend, frames, width, rows):
    """QuantizedAvxChecks.cs:17-50 through TryQuantizedLinear, bit-exact to
    the committed golden outputs (fp32 scale plane: 0.013/-0.007 are not fp16)."""
    from funasrnet_amd.model import Q8Tensor
    values, w, ws, bias, _ = q8_kat_case(frames, width, rows)
    golden = np.load(os.path.join(GOLDEN, "q8_kat.npz"))[f"{frames}x{width}x{rows}"]
    out = np.full(frames * rows, 123.0, dtype=np.float32)
    assert backend.try_quantized_linear(values, frames, Q8Tensor("kat", w, ws), bias, out)
    assert np.array_equal(out.reshape(frames, rows).view(np.uint32), golden.view(np.uint32))


def test_linear_many_equals_independent(backend, oracle_lib):
    """QuantizedGroupAvxChecks.cs:17-85: grouped outputs bit-identical to
    separate projections and to the oracle, signed/zero scales, -128 weights."""
    from funasrnet_amd.model import Q8Tensor
    rng = np.random.default_rng(512031)
    for frames in (1, 2, 5, 17):
        for width in (32, 96, 1024):
            x = rng.standard_normal(frames * width).astype(np.float32)
            tensors = []
            for rows in (1, 3, 17, 32, 65):
                q = np.where(np.arange(rows * width).reshape(rows, width) % 5 == 0, -128,
                             rng.integers(-127, 128, (rows, width))).astype(np.int8)
                s = np.array([0.0, -0.007, 0.013, 0.125], dtype=np.float32)[np.arange(rows * width // 32) % 4]
                tensors.append(Q8Tensor(f"g{rows}", q, s.reshape(rows, -1)))
            outs = backend.try_linear_many(x, frames, tensors)
            assert outs is not None
            for t, o in zip(tensors, outs):
                single = np.empty(frames * t.rows, dtype=np.float32)
                assert backend.try_quantized_linear(x, frames, t, None, single)
                expected = oracle_lib.linear(x, t.quantized, t.scales).ravel()
                assert np.array_equal(o.view(np.uint32), single.view(np.uint32))
                assert np.array_equal(o.view(np.uint32), expected.view(np.uint32))


@pytest.mark.parametrize("frames", [1, 3])
def test_quantized_linear_wide_input(backend, oracle_lib, frames):
    """The seam's Q8_0 linear at K = 6144 (past the four register chunks of
    the decoder's widths): the oracle's quantise-then-GEMV bits."""
    rng = np.random.default_rng(61 + frames)
    w = _weights(rng, 2048, 6144)
    x = rng.standard_normal((frames, 6144)).astype(np.float32)
    out = np.zeros((frames, 2048), dtype=np.float32)
    assert backend.try_quantized_linear(x.ravel(), frames, w, None, out.ravel())
    for f in range(frames):
        xq, xs = oracle_lib.quantize(x[f])
        expected = oracle_lib.gemv_quantized(xq, xs, w.quantized, w.scales)[0]
        assert np.array_equal(out[f].view(np.uint32), expected.view(np.uint32)), f


def test_declines_small_and_leaves_output_untouched():
    """IQuantizedComputeBackend contract: a declined call returns false and
    the output keeps its contents (MinimumOperations, VulkanFloatBackend.cs:36)."""
    from funasrnet_amd.hip import HipBackend
    from funasrnet_amd.model import Q8Tensor
    b = HipBackend(0)  # default minimum of 250000 multiply-adds
    try:
        w = Q8Tensor("tiny", np.ones((3, 32), dtype=np.int8), np.ones((3, 1), dtype=np.float32))
        out = np.full(3, 123.0, dtype=np.float32)
        assert not b.try_quantized_linear(np.ones(32, dtype=np.float32), 1, w, None, out)
        assert np.all(out == 123.0)
        with pytest.raises(ValueError):
            b.try_quantized_linear(np.ones(31, dtype=np.float32), 1, w, None, out)
    finally:
        b.close()


@pytest.mark.parametrize("cols,rows", [(1024, 2048), (3072, 1024)])
def test_gguf_block_upload_equals_unpacked_upload(backend, dev, oracle_lib, cols, rows):
    """fah_weight_q8_upload_blocks: the GGUF blocks split on the device give
    the same weight as the host-unpacked planes (identical GEMV bits), with
    every fp16 scale pattern class present (normal, subnormal, zero, -0)."""
    from funasrnet_amd import gguf
    from funasrnet_amd.model import Q8Tensor
    rng = np.random.default_rng(rows + cols)
    w = _weights(rng, rows, cols)
    bits = w.scales.astype(np.float16).view(np.uint16).reshape(-1).copy()
    bits[:4] = [0x0001, 0x0000, 0x8000, 0x03FF]  # subnormals, +0, -0
    raw = np.frombuffer(gguf.pack_q8_0(w.quantized, bits), dtype=np.uint8)
    q, s, _ = gguf.unpack_q8_0(raw, rows * cols // 32)
    arrays = Q8Tensor("w", q.reshape(rows, cols), s.reshape(rows, -1))
    blocks = Q8Tensor("w", None, None, blocks=raw, dims=(rows, cols))
    ha, hb = backend.weight(arrays), backend.weight(blocks)
    assert ha.device_bytes == hb.device_bytes
    x = rng.standard_normal(cols).astype(np.float32)
    xq, xs = oracle_lib.quantize(x)
    dq, ds = dev.DeviceArray.from_numpy(xq), dev.DeviceArray.from_numpy(xs)
    oa, ob = dev.DeviceArray(rows, np.float32), dev.DeviceArray(rows, np.float32)
    backend.gemv_device(dq.ptr, ds.ptr, 1, ha, oa.ptr)
    backend.gemv_device(dq.ptr, ds.ptr, 1, hb, ob.ptr)
    backend.synchronize()
    assert np.array_equal(oa.numpy().view(np.uint32), ob.numpy().view(np.uint32))
    expected = oracle_lib.gemv_quantized(xq, xs, arrays.quantized, arrays.scales)[0]
    assert np.array_equal(ob.numpy().view(np.uint32), expected.view(np.uint32))
    ha.close()
    hb.close()

"""The FP32 seam on the device against the oracle's double references, with
the reference's own device-check shapes and tolerances
(tools/FunAsrNet.Benchmarks/FloatGpuChecks.cs, AttentionGpuChecks.cs,
Program.cs ReLU chain checks): TryLinear within 2e-4 x max(1, |expected|),
a group bit-identical to separate calls, the ReLU chain bit-identical to its
two projections, attention within 5e-5, declines leaving the output
untouched."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def backend():
    from funasrnet_amd.hip import HipBackend
    b = HipBackend(0, minimum_operations=0)
    yield b
    b.close()


def _close(got, expected, tol):
    err = np.abs(got.astype(np.float64) - expected) / np.maximum(1.0, np.abs(expected))
    assert np.all(np.isfinite(got)) and err.max() <= tol, err.max()


@pytest.mark.parametrize("frames", [1, 3, 17, 33])
@pytest.mark.parametrize("width", [19, 65, 513, 1024, 1057, 3073])
def test_linear_and_group(backend, oracle_lib, frames, width):
    rng = np.random.default_rng(211109 + frames * 7 + width)
    x = (rng.random((frames, width)) - 0.5).astype(np.float32)
    weights = [(rng.random((rows, width)) - 0.5).astype(np.float32) for rows in (7, 65, 129)]
    grouped = backend.try_linear_many(x, frames, weights)
    assert grouped is not None
    for w, g in zip(weights, grouped):
        out = np.full(frames * w.shape[0], np.nan, np.float32)
        assert backend.try_linear(x, frames, w, None, out)
        assert np.array_equal(g.view(np.uint32), out.view(np.uint32))
        _close(out.reshape(frames, -1), oracle_lib.float_linear_f64(x, frames, w), 2e-4)
    # Again after other uploads: the same bits.
    again = backend.try_linear_many(x, frames, weights)
    for g, a in zip(grouped, again):
        assert np.array_equal(g.view(np.uint32), a.view(np.uint32))


def test_linear_bias_and_decoder_gemv_shapes(backend, oracle_lib):
    rng = np.random.default_rng(7)
    for frames, cols, rows in [(1, 1024, 2048), (1, 3072, 1024), (2, 1024, 6144), (64, 560, 1536), (150, 512, 2048),
                               (1000, 512, 1536), (1000, 2048, 512), (257, 516, 100), (5, 36, 70)]:
        x = rng.standard_normal((frames, cols)).astype(np.float32)
        w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        b = rng.standard_normal(rows).astype(np.float32)
        out = np.empty(frames * rows, np.float32)
        assert backend.try_linear(x, frames, w, b, out)
        _close(out.reshape(frames, rows), oracle_lib.float_linear_f64(x, frames, w, b), 2e-4)


@pytest.mark.parametrize("shape", [(1, 19, 32, 7), (33, 65, 64, 35), (3, 19, 32, 19), (3, 513, 512, 513),
                                   (1, 513, 512, 509), (100, 512, 2048, 512)])
def test_relu_projection_equals_two_projections(backend, oracle_lib, shape):
    M, K, H, N = shape
    rng = np.random.default_rng(M * 1000 + K)
    first = (rng.random((H, K)) - 0.5).astype(np.float32)
    second = (rng.random((N, H)) - 0.5).astype(np.float32)
    b1 = (rng.random(H) - 0.5).astype(np.float32)
    b2 = (rng.random(N) - 0.5).astype(np.float32)
    x = (rng.random((M, K)) - 0.5).astype(np.float32)
    for with_bias in (False, True):
        mid = np.empty(M * H, np.float32)
        assert backend.try_linear(x, M, first, b1 if with_bias else None, mid)
        mid = np.where(mid < 0, np.float32(0), mid)
        expected = np.empty(M * N, np.float32)
        assert backend.try_linear(mid, M, second, b2 if with_bias else None, expected)
        got = np.full(M * N, np.nan, np.float32)
        assert backend.try_relu_projection(x, M, first, b1 if with_bias else None, second,
                                           b2 if with_bias else None, got)
        assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))
        ref_mid = np.maximum(oracle_lib.float_linear_f64(x, M, first, b1 if with_bias else None), 0.0)
        ref = ref_mid @ second.astype(np.float64).T + (b2.astype(np.float64) if with_bias else 0.0)
        _close(got.reshape(M, N), ref, 1e-3)


def test_relu_projection_declines(backend):
    rng = np.random.default_rng(9)
    first = rng.random((30, 19)).astype(np.float32)  # 30 rows: not a multiple of 4
    second = rng.random((7, 30)).astype(np.float32)
    out = np.full(7, 123.0, np.float32)
    assert not backend.try_relu_projection(rng.random(19).astype(np.float32), 1, first, None, second, None, out)
    assert np.all(out == 123.0)


@pytest.mark.parametrize("frames,width,heads", [(1, 7, 1), (2, 7, 1), (3, 256, 1), (17, 96, 3), (100, 512, 4),
                                                (129, 1024, 8), (400, 512, 4), (257, 256, 1), (1024, 16, 2),
                                                (1025, 16, 2), (4096, 8, 1), (1, 128, 1), (33, 512, 8),
                                                (300, 256, 4), (1000, 512, 4)])
def test_attention(backend, oracle_lib, frames, width, heads):
    rng = np.random.default_rng(170719 + frames + width)
    q = (rng.random((frames, width)) * 2 - 1).astype(np.float32)
    k = (rng.random((frames, width)) * 2 - 1).astype(np.float32)
    v = (rng.random((frames, width)) * 8 - 4).astype(np.float32)
    if frames == 17:
        q *= 16
        k *= 16
    out = np.full(frames * width, np.nan, np.float32)
    assert backend.try_attention(q, k, v, frames, width, heads, out)
    _close(out.reshape(frames, width), oracle_lib.attention_f64(q, k, v, frames, width, heads), 5e-5)
    # Zero queries and keys: every row is the mean of the values.
    z = np.zeros_like(q)
    assert backend.try_attention(z, z, v, frames, width, heads, out)
    mean = v.astype(np.float64).mean(axis=0)
    _close(out.reshape(frames, width), np.broadcast_to(mean, (frames, width)), 5e-5)


def test_attention_declines_unsupported_shapes(backend):
    from funasrnet_amd import hip
    import ctypes
    lib = hip.load()
    sentinel = np.array([123.0], np.float32)
    fp = ctypes.POINTER(ctypes.c_float)
    dummy = np.zeros(8, np.float32)
    for frames, width, heads in [(4097, 8, 1), (1, 257, 1), (4, 10, 3)]:
        rc = lib.fah_attention(backend.handle, dummy.ctypes.data_as(fp), dummy.ctypes.data_as(fp),
                               dummy.ctypes.data_as(fp), frames, width, heads, sentinel.ctypes.data_as(fp))
        assert rc == hip.DECLINED and sentinel[0] == 123.0

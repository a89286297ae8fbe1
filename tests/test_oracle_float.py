"""Pins of the oracle's double references for the FP32 seam (projections,
ReLU chains and non-causal attention) by checks that do not restate them:
exact integer brute force, numpy's float64 matmul, and closed forms of
attention (the reference's own AttentionGpuChecks.cs uses q = k = 0 -> the
mean of v)."""
import numpy as np
import pytest


def test_linear_integer_inputs_exact(oracle_lib):
    rng = np.random.default_rng(1)
    for frames, cols, rows in [(1, 19, 7), (3, 65, 129), (17, 513, 33)]:
        x = rng.integers(-8, 9, size=(frames, cols))
        w = rng.integers(-8, 9, size=(rows, cols))
        b = rng.integers(-100, 101, size=rows)
        got = oracle_lib.float_linear_f64(x.astype(np.float32), frames, w.astype(np.float32), b.astype(np.float32))
        assert np.array_equal(got, (x.astype(np.int64) @ w.T.astype(np.int64) + b).astype(np.float64))


def test_linear_random_vs_numpy_float64(oracle_lib):
    rng = np.random.default_rng(2)
    frames, cols, rows = 9, 1057, 65
    x = (rng.random((frames, cols)) - 0.5).astype(np.float32)
    w = (rng.random((rows, cols)) - 0.5).astype(np.float32)
    got = oracle_lib.float_linear_f64(x, frames, w)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.abs(got - ref).max() <= 1e-12 * max(1.0, np.abs(ref).max())


def test_linear_identity_and_zero_weights(oracle_lib):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 32)).astype(np.float32)
    b = rng.standard_normal(32).astype(np.float32)
    got = oracle_lib.float_linear_f64(x, 4, np.eye(32, dtype=np.float32), b)
    assert np.array_equal(got, x.astype(np.float64) + b.astype(np.float64))
    assert np.array_equal(oracle_lib.float_linear_f64(x, 4, np.zeros((5, 32), np.float32), b[:5]),
                          np.broadcast_to(b[:5].astype(np.float64), (4, 5)))


def test_attention_zero_queries_give_the_mean_of_values(oracle_lib):
    rng = np.random.default_rng(4)
    for frames, width, heads in [(1, 7, 1), (17, 96, 3), (100, 64, 4)]:
        z = np.zeros((frames, width), np.float32)
        v = (rng.random((frames, width)) * 8 - 4).astype(np.float32)
        got = oracle_lib.attention_f64(z, z, v, frames, width, heads)
        mean = v.astype(np.float64).mean(axis=0)
        assert np.abs(got - mean).max() <= 1e-12 * max(1.0, np.abs(mean).max())


def test_attention_single_frame_and_dominant_key(oracle_lib):
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 16)).astype(np.float32)
    v = rng.standard_normal((1, 16)).astype(np.float32)
    assert np.allclose(oracle_lib.attention_f64(q, q, v, 1, 16, 2), v.astype(np.float64), rtol=0, atol=1e-15)
    # One key far along the query: its value wins for every query.
    frames, width = 8, 8
    q = np.ones((frames, width), np.float32)
    k = np.zeros((frames, width), np.float32)
    k[5] = 100.0
    v = rng.standard_normal((frames, width)).astype(np.float32)
    got = oracle_lib.attention_f64(q, k, v, frames, width, 1)
    assert np.allclose(got, np.broadcast_to(v[5].astype(np.float64), (frames, width)), rtol=0, atol=1e-12)


def test_attention_heads_independent_and_key_permutation(oracle_lib):
    rng = np.random.default_rng(6)
    frames, width, heads = 13, 24, 3
    q, k, v = (rng.standard_normal((frames, width)).astype(np.float32) for _ in range(3))
    full = oracle_lib.attention_f64(q, k, v, frames, width, heads)
    size = width // heads
    for h in range(heads):
        sl = slice(h * size, (h + 1) * size)
        alone = oracle_lib.attention_f64(np.ascontiguousarray(q[:, sl]), np.ascontiguousarray(k[:, sl]),
                                         np.ascontiguousarray(v[:, sl]), frames, size, 1)
        assert np.array_equal(alone, full[:, sl])
    perm = rng.permutation(frames)
    shuffled = oracle_lib.attention_f64(q, k[perm], v[perm], frames, width, heads)
    assert np.abs(shuffled - full).max() <= 1e-12

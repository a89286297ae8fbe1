"""Pins the oracle's element-wise and reduction functions: exhaustive binary16
tables, closed forms, and double-precision references at the reference's own
tolerances (tests/FunAsrNet.Checks/Program.cs:297-363, FrontendKernelChecks.cs)."""
import math

import numpy as np
import pytest

f32 = np.float32


def _all_half_values():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    return bits.view(np.float16)


def test_half_to_float_exhaustive(oracle_lib):
    h = _all_half_values()
    got = np.array([oracle_lib.half_to_float(int(b)) for b in h.view(np.uint16)], dtype=np.float32)
    finite = ~np.isnan(h)
    assert np.array_equal(got[finite].view(np.uint32), h[finite].astype(np.float32).view(np.uint32))
    assert np.isnan(got[~finite]).all()


def test_round_half_exhaustive_and_midpoints(oracle_lib):
    """Program.cs:366-398: every binary16 value, each rounding midpoint and its
    +-1 ulp neighbours, both signs; expected = numpy's RNE float16 cast."""
    h = _all_half_values()
    vals = [h.astype(np.float32)]
    finite = h[:0x7BFF + 1].astype(np.float32)  # 0 .. 65504 positive
    nxt = h[1:0x7BFF + 2].astype(np.float32)
    mid = ((finite + nxt) * f32(0.5)).astype(np.float32)
    for m in (mid, np.nextafter(mid, f32(np.inf)), np.nextafter(mid, f32(-np.inf))):
        vals += [m, -m]
    rng = np.random.default_rng(5)
    vals.append(rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32))
    x = np.concatenate(vals)
    x = x[~np.isnan(x)]
    got = oracle_lib.round_half(x)
    with np.errstate(over="ignore"):
        expected = x.astype(np.float16).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))
    assert np.isnan(oracle_lib.round_half(np.array([np.nan], dtype=np.float32))).all()


def test_exp_close_to_double(oracle_lib):
    """ExpAvx (TensorMath.ExpAvx.cs:83-116) evaluates in double: within 1 ulp of
    the correctly rounded float exp, exact at 0, saturating outside +-104."""
    x = np.concatenate([np.linspace(-103.9, 88.7, 20001), np.random.default_rng(1).standard_normal(5000) * 10]).astype(np.float32)
    got = oracle_lib.exp(x)
    ref = np.exp(x.astype(np.float64)).astype(np.float32)
    ulp = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert ulp.max() <= 1
    assert (ulp == 0).mean() > 0.99
    assert oracle_lib.exp(np.array([0.0, -0.0, -1e9, 1e9], dtype=np.float32)).tolist() == [1.0, 1.0, 0.0, np.inf]
    assert np.isnan(oracle_lib.exp(np.array([np.nan], dtype=np.float32))[0])


@pytest.mark.parametrize("width", [1, 3, 4, 7, 8, 17, 128, 512, 1024])
def test_rms_norm_vs_double(oracle_lib, width):
    """Program.cs:297-335 (rms branch): within 1e-5 * max(1, |ref|) of double."""
    rng = np.random.default_rng(width)
    x = (rng.random(width * 3) * 20 - 10).astype(np.float32)
    scale = rng.random(width).astype(np.float32)
    got = oracle_lib.rms_norm(x, width, scale, 1e-5)
    xd = x.astype(np.float64).reshape(3, width)
    ref = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-5) * scale
    assert np.all(np.abs(got.reshape(3, width) - ref) <= 1e-5 * np.maximum(1, np.abs(ref)))


def test_rms_norm_lane_order(oracle_lib):
    """The double sum of squares pairs lanes as (s0+s2)+(s1+s3); a value
    whose float result depends on that order pins it."""
    x = np.zeros(8, dtype=np.float32)
    x[0], x[1], x[2], x[3] = 2.0 ** 26, 1.0, -(2.0 ** 26), 1.0  # squares 2^52, 1, 2^52, 1
    x[4] = 1.0
    got = oracle_lib.rms_norm(x, 8, np.ones(8, dtype=np.float32), 0.0)
    s0, s1, s2, s3 = 2.0 ** 52 + 1.0, 1.0, 2.0 ** 52, 1.0
    variance = (s0 + s2) + (s1 + s3)
    inverse = f32(1) / f32(math.sqrt(f32(variance / 8)))
    assert got[4] == f32(f32(1.0) * inverse)


@pytest.mark.parametrize("width", [1, 3, 4, 7, 8, 17, 128, 512, 1024])
@pytest.mark.parametrize("amplitude", [0.0, 1.0, 50.0])
def test_softmax_vs_double(oracle_lib, width, amplitude):
    """Program.cs:337-355: within 5e-7 of double, sums to 1 within 1e-6."""
    rng = np.random.default_rng(width)
    x = ((rng.random(width) * 20 - 10) * amplitude).astype(np.float32)
    got = oracle_lib.softmax(x)
    xd = x.astype(np.float64)
    ref = np.exp(xd - xd.max()) / np.exp(xd - xd.max()).sum()
    assert np.all(np.abs(got - ref) <= 5e-7 * np.maximum(1, np.abs(ref)))
    assert abs(float(got.astype(np.float64).sum()) - 1) <= 1e-6


def test_silu_multiply_vs_double(oracle_lib):
    """Program.cs:357-363: within 2e-6."""
    rng = np.random.default_rng(2)
    x = (rng.random(3 * 1024) * 20 - 10).astype(np.float32)
    up = (x * f32(0.1)).astype(np.float32)
    got = oracle_lib.silu_multiply(x, up)
    xd = x.astype(np.float64)
    ref = xd / (1 + np.exp(-xd)) * up
    assert np.all(np.abs(got - ref) <= 2e-6 * np.maximum(1, np.abs(ref)))


@pytest.mark.parametrize("half", list(range(0, 34)) + [63, 64, 65, 128])
def test_rotate_half_closed_form(oracle_lib, half):
    """FrontendKernelChecks.cs:54-71: a*c - b*s and a*s + b*c per pair,
    product-then-add with no fused multiply-add, including -0, eps, max."""
    rng = np.random.default_rng(half)
    cos = np.cos(np.arange(half)).astype(np.float32)
    sin = np.sin(np.arange(half)).astype(np.float32)
    x = (rng.random(2 * half) * 20 - 10).astype(np.float32)
    for i in range(0, 2 * half, 7):
        x[i] = (-0.0, 1.4e-45, np.finfo(np.float32).max)[i % 3]
    got = oracle_lib.rotate_half(x, cos, sin) if half else x
    a, b = x[:half], x[half:]
    with np.errstate(over="ignore", invalid="ignore"):
        exp = np.concatenate([(a * cos).astype(np.float32) - (b * sin).astype(np.float32),
                              (a * sin).astype(np.float32) + (b * cos).astype(np.float32)]).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_rope_table_vs_double(oracle_lib):
    """QwenDecoder.cs:78-95 with glibc powf/cosf/sinf: the bits follow the C
    runtime; checked here against double evaluation of the same float angle."""
    c, s = oracle_lib.rope_table(4224, 128, 1e6)
    i = np.arange(64)
    freq = np.array([f32(np.power(f32(1e6), f32(f32(-2.0 * k) / f32(128)))) for k in i], dtype=np.float32)
    angle = (np.arange(4224, dtype=np.float32)[:, None] * freq[None, :]).astype(np.float32)
    # numpy's float32 power may differ from glibc powf by an ulp, which moves
    # the float angle by up to an ulp of itself: allow that much slack.
    slack = 2e-7 + angle.astype(np.float64) * 2.0 ** -22
    assert np.all(np.abs(c - np.cos(angle.astype(np.float64))) <= slack)
    assert np.all(np.abs(s - np.sin(angle.astype(np.float64))) <= slack)
    assert np.all(c[0] == 1) and np.all(s[0] == 0)
    assert np.all(np.abs(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2 - 1) <= 4e-7)


def _reference_greedy(values):
    best = 0
    for i in range(1, len(values)):
        if values[i] > values[best]:
            best = i
    return best


@pytest.mark.parametrize("length", list(range(0, 66)) + [4097])
def test_greedy_patterns(oracle_lib, length):
    """FrontendKernelChecks.cs:72-121: strict '>' scan, first max wins, NaN
    never wins, a NaN first element returns 0, -0 equals +0."""
    rng = np.random.default_rng(length)
    i = np.arange(length)
    kinds = [
        (rng.random(length) - 0.5),
        i.astype(float), -i.astype(float), np.full(length, -np.inf),
        np.where(i % 3 == 0, np.nan, np.where(i % 3 == 1, np.inf, 0.0)),
        np.where(i == 0, -1.0, np.where(i % 7 == 0, 1.0, np.nan)),
        np.where(i % 2 == 0, -0.0, 0.0),
        np.where(i % 3 == 0, -np.inf, np.nan),
    ]
    for v in kinds:
        v = np.asarray(v, dtype=np.float32)
        assert oracle_lib.greedy(v) == _reference_greedy(v.tolist())


def test_greedy_vocab_size(oracle_lib):
    v = np.random.default_rng(0).standard_normal(151936).astype(np.float32)
    v[151935] = v.max()  # tie: first occurrence wins
    assert oracle_lib.greedy(v) == int(np.argmax(v))


def test_dot_lane_order(oracle_lib):
    """AudioKernels.Dot: eight lane accumulators folded as
    ((a0+a4)+(a1+a5))+((a2+a6)+(a3+a7)); a sequential dot differs here."""
    a = np.zeros(16, dtype=np.float32)
    b = np.ones(16, dtype=np.float32)
    a[0], a[1], a[4], a[5] = 2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)
    # lanes: a0=2^24, a1=1, a4=1, a5=-2^24 -> b0=2^24+1->2^24, b1=1-2^24 -> sum 1
    assert oracle_lib.dot(a, b) == 1.0
    seq = f32(0)
    for v in a:
        seq = f32(seq + v)
    assert seq != 1.0


def test_attention_vs_float64(oracle_lib):
    """AttentionGpuChecks.cs:113-156 tolerance (5e-5) for causal GQA."""
    rng = np.random.default_rng(4)
    heads, kv, hs, frames, position = 4, 2, 128, 3, 20
    end = position + frames
    q = rng.standard_normal(frames * heads * hs).astype(np.float32)
    k = rng.standard_normal(end * kv * hs).astype(np.float32)
    v = rng.standard_normal(end * kv * hs).astype(np.float32)
    got = oracle_lib.attention(q, k, v, frames, position, heads, kv, hs).reshape(frames, heads, hs)
    qd = q.astype(np.float64).reshape(frames, heads, hs)
    kd = k.astype(np.float64).reshape(end, kv, hs)
    vd = v.astype(np.float64).reshape(end, kv, hs)
    for t in range(frames):
        for h in range(heads):
            n = position + t + 1
            s = kd[:n, h // 2] @ qd[t, h] / math.sqrt(hs)
            p = np.exp(s - s.max())
            p /= p.sum()
            ref = p @ vd[:n, h // 2]
            assert np.all(np.abs(got[t, h] - ref) <= 5e-5)


def test_attention_values_sequential(oracle_lib):
    """Program.cs:400-431: the value sum equals repeated AddScaled in time
    order (out += v_t * p_t from 0f)."""
    rng = np.random.default_rng(9)
    hs, n = 128, 37
    q = rng.standard_normal(hs).astype(np.float32)
    k = rng.standard_normal(n * hs).astype(np.float32)
    v = rng.standard_normal(n * hs).astype(np.float32)
    got = oracle_lib.attention(q, k, v, 1, n - 1, 1, 1, hs)
    scores = np.array([oracle_lib.dot(q, k[t * hs:(t + 1) * hs]) / f32(math.sqrt(hs)) for t in range(n)], dtype=np.float32)
    p = oracle_lib.softmax(scores)
    acc = np.zeros(hs, dtype=np.float32)
    for t in range(n):
        acc = (acc + (v[t * hs:(t + 1) * hs] * p[t]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), acc.view(np.uint32))

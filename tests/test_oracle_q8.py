"""Pins the oracle's activation quantiser and Q8_0 projection against the
reference's known-answer tests, closed forms and brute force."""
import os

import numpy as np
import pytest

from tests.golden.make_golden import q8_kat_case, quantize_reference

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
f32 = np.float32


def test_quantize_halfway_closed_form(oracle_lib):
    """QuantizeRoundingChecks.cs:83-87: with max 127 the scale is exactly 1, so
    q(v+0.5) rounds away from zero and the +-1 ulp neighbours round to the
    nearer integer."""
    for v in range(-126, 127):
        h = f32(v + 0.5)
        block = np.zeros(32, dtype=np.float32)
        block[:4] = [127, h, np.nextafter(h, f32(-np.inf)), np.nextafter(h, f32(np.inf))]
        q, s = oracle_lib.quantize(block)
        assert s[0] == 1.0
        away = v + 1 if v >= 0 else v
        assert list(q[:4]) == [127, away, v, v + 1], v
        assert not q[4:].any()


def test_quantize_specials_closed_form(oracle_lib):
    """QuantizeRoundingChecks.cs:93-95 specials at index 17."""
    def block(value):
        b = np.zeros(32, dtype=np.float32)
        b[17] = value
        return oracle_lib.quantize(b)

    for z in (0.0, -0.0):
        q, s = block(z)
        assert s[0] == 0 and not np.signbit(s[0]) and not q.any()
    q, s = block(1.4e-45)  # epsilon / 127 underflows to zero
    assert s[0] == 0 and not q.any()
    q, s = block(np.finfo(np.float32).max)
    assert s[0] == f32(np.finfo(np.float32).max / f32(127)) and q[17] == 127 and np.count_nonzero(q) == 1
    q, s = block(np.nan)
    assert np.isnan(s[0]) and not q.any()
    for inf in (np.inf, -np.inf):
        q, s = block(inf)
        assert s[0] == np.inf and not q.any()


def test_quantize_overflowing_inverse_closed_form(oracle_lib):
    """A block whose scale is subnormal has an infinite inverse: nonzero
    values saturate to +-127, zeros stay 0 (0*inf is NaN, which converts to 0)."""
    tiny = f32(np.ldexp(1.0, -140))
    block = np.array([((i * 7) % 15 - 7) * tiny for i in range(32)], dtype=np.float32)
    q, s = oracle_lib.quantize(block)
    assert s[0] == f32(f32(7 * tiny) / f32(127))
    assert np.isinf(f32(1) / s[0])
    assert np.array_equal(q, np.sign(block).astype(np.int8) * 127)


def test_quantize_matches_golden(oracle_lib):
    g = np.load(os.path.join(GOLDEN, "quantize_kat.npz"))
    q, s = oracle_lib.quantize(g["input"])
    assert np.array_equal(q, g["q"])
    assert np.array_equal(np.isnan(s), np.isnan(g["scales"]))
    ok = ~np.isnan(s)
    assert np.array_equal(s[ok].view(np.uint32), g["scales"][ok].view(np.uint32))


def test_quantize_random_vs_fraction_rounding(oracle_lib):
    """Random N(0,1) and wide-range blocks vs the Fraction-based restatement."""
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.standard_normal(32 * 64), rng.standard_normal(32 * 64) * 10.0 ** rng.integers(-30, 30, 32 * 64)])
    x = x.astype(np.float32)
    q, s = oracle_lib.quantize(x)
    q2, s2 = quantize_reference(x)
    assert np.array_equal(q, q2)
    assert np.array_equal(s.view(np.uint32), s2.view(np.uint32))
    assert q.min() >= -127 and q.max() <= 127


def test_quantize_rejects_partial_block(oracle_lib):
    with pytest.raises(ValueError):
        oracle_lib.quantize(np.zeros(31, dtype=np.float32))


def test_block_dot_brute_force(oracle_lib):
    """Exact int32 dot including -128 weights (QuantizedAvxChecks.cs:29)."""
    rng = np.random.default_rng(3)
    w = rng.integers(-128, 128, size=(19, 96), dtype=np.int8)
    x = rng.integers(-127, 128, size=96, dtype=np.int8)
    dots = oracle_lib.block_dots(x, w)
    expected = (w.astype(np.int64).reshape(19, 3, 32) * x.astype(np.int64).reshape(1, 3, 32)).sum(-1)
    assert np.array_equal(dots, expected)
    extreme = np.full((1, 32), -128, dtype=np.int8)
    assert oracle_lib.block_dots(np.full(32, -127, dtype=np.int8), extreme)[0, 0] == 32 * 128 * 127


@pytest.mark.parametrize("frames", [1, 3, 17])
@pytest.mark.parametrize("width", [32, 96, 1024])
@pytest.mark.parametrize("rows", [1, 3, 19, 32])
def test_q8_linear_reference_kat(oracle_lib, frames, width, rows):
    """QuantizedAvxChecks.cs:17-50, bit-exact against the golden fixture."""
    values, w, ws, bias, _ = q8_kat_case(frames, width, rows)
    golden = np.load(os.path.join(GOLDEN, "q8_kat.npz"))[f"{frames}x{width}x{rows}"]
    out = oracle_lib.linear(values, w, ws, bias)
    assert np.array_equal(out.view(np.uint32), golden.view(np.uint32))


def test_q8_block_order_is_sequential(oracle_lib):
    """Block products [2^24, 1, 1, -2^24] sum to 0 only left to right from 0f:
    a pairwise sum gives 1 and a reversed sum 2, so a changed float order
    (tree, reversed, scales multiplied first) fails here."""
    xq = np.ones(128, dtype=np.int8)
    xs = np.ones(4, dtype=np.float32)
    w = np.ones((1, 128), dtype=np.int8)
    ws = np.array([[2.0 ** 19, 2.0 ** -5, 2.0 ** -5, -(2.0 ** 19)]], dtype=np.float32)
    assert oracle_lib.gemv_quantized(xq, xs, w, ws)[0, 0] == 0.0
    # (dot * ws) * xs, not dot * (ws * xs): with ws = 1.5*2^-75, xs = 2^-75 the
    # first order is exact (24 * 2^-149 per block), the second rounds
    # ws*xs = 0.75 * 2^-149 up to 2^-149 and gives 32 * 2^-149 per block.
    xs_tiny = np.full(4, 2.0 ** -75, dtype=np.float32)
    ws_tiny = np.full((1, 4), 1.5 * 2.0 ** -75, dtype=np.float32)
    got = oracle_lib.gemv_quantized(xq, xs_tiny, w, ws_tiny)[0, 0]
    assert got == np.float32(96 * 2.0 ** -149)


def test_grouped_equals_independent(oracle_lib):
    """QuantizedGroupAvxChecks.cs:52-53: one shared quantisation gives the same
    bits as separate projections; also equals the brute-force formula."""
    rng = np.random.default_rng(11)
    width = 96
    x = rng.standard_normal((5, width)).astype(np.float32)
    mats = []
    for rows in (1, 3, 17, 32, 65):
        w = np.where(np.arange(rows * width).reshape(rows, width) % 5 == 0, -128,
                     rng.integers(-127, 128, (rows, width))).astype(np.int8)
        ws = np.array([0.0, -0.007, 0.013, 0.125], dtype=np.float32)[np.arange(rows * width // 32) % 4].reshape(rows, -1)
        mats.append((w, ws))
    q, s = oracle_lib.quantize(x.ravel())
    for w, ws in mats:
        grouped = oracle_lib.gemv_quantized(q, s, w, ws)
        independent = oracle_lib.linear(x, w, ws)
        assert np.array_equal(grouped.view(np.uint32), independent.view(np.uint32))
        dots = np.einsum("tbk,rbk->trb", q.reshape(5, 3, 32).astype(np.int64), w.reshape(-1, 3, 32).astype(np.int64))
        for t in range(5):
            for r in range(w.shape[0]):
                acc = f32(0)
                for b in range(3):
                    acc = f32(acc + f32(f32(f32(dots[t, r, b]) * ws[r, b]) * s[t * 3 + b]))
                assert grouped[t, r].view(np.uint32) == f32(acc).view(np.uint32)


def test_unpack_q8_exhaustive_scales(oracle_lib):
    """Q8ModelLoadingChecks.cs:13-36: all 65536 fp16 scale patterns and the
    payload pattern (block*17 + i*31) & 255."""
    blocks = 65536
    raw = np.zeros((blocks, 34), dtype=np.uint8)
    b = np.arange(blocks)
    raw[:, 0] = b & 0xFF
    raw[:, 1] = b >> 8
    raw[:, 2:] = ((b[:, None] * 17 + np.arange(32)[None, :] * 31) & 255).astype(np.uint8)
    q, s = oracle_lib.unpack_q8(raw.ravel(), blocks)
    assert np.array_equal(q.view(np.uint8), raw[:, 2:].ravel())
    half = b.astype(np.uint16).view(np.float16)
    finite = ~np.isnan(half)
    assert np.array_equal(s[finite].view(np.uint32), half[finite].astype(np.float32).view(np.uint32))
    nan_bits = s[~finite].view(np.uint32)
    hb = b[~finite].astype(np.uint32)
    assert np.array_equal(nan_bits, ((hb & 0x8000) << 16) | 0x7FC00000 | ((hb & 0x3FF) << 13))

"""Writes the golden fixtures in this folder from the reference's own
deterministic known-answer inputs, with expected outputs computed by an
independent numpy/fractions restatement (not by the C oracle, not by the HIP
library).

  quantize_kat.npz  TensorMath.Quantize cases of
                    tests/FunAsrNet.Checks/QuantizeRoundingChecks.cs:83-95
                    (halfway +-1 ulp for every integer -126..126, specials) and
                    Program.cs:270-295 (amplitude sweep), plus denormal-scale
                    blocks in the spirit of QuantizeRoundingChecks.cs:88-92.
  q8_kat.npz        TensorMath.Linear Q8 cases of
                    tests/FunAsrNet.Checks/QuantizedAvxChecks.cs:17-50:
                    frames {1,3,17} x width {32,96,1024} x rows {1,3,19,32}.

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
f32 = np.float32


def round_away(v: np.float32) -> int:
    """MathF.Round(v, AwayFromZero) then .NET 9+ saturating (int) cast."""
    if np.isnan(v):
        return 0
    if np.isinf(v):
        return 2**31 - 1 if v > 0 else -2**31
    fr = Fraction(float(v))
    mag = abs(fr)
    n = int(mag)  # floor of magnitude
    if mag - n >= Fraction(1, 2):
        n += 1
    n = n if fr >= 0 else -n
    return max(-2**31, min(2**31 - 1, n))


def quantize_reference(x: np.ndarray):
    """Scalar statement of TensorMath.cs:397-411 with Fraction rounding."""
    x = x.astype(np.float32)
    q = np.zeros(x.size, dtype=np.int8)
    s = np.zeros(x.size // 32, dtype=np.float32)
    with np.errstate(all="ignore"):
        for b in range(x.size // 32):
            block = x[b * 32:(b + 1) * 32]
            m = f32(0)
            for v in block:
                a = f32(abs(v))
                if np.isnan(m):
                    continue
                m = a if (np.isnan(a) or a > m) else m
            d = f32(m / f32(127))
            inv = f32(0) if d == 0 else f32(f32(1) / d)
            s[b] = d
            for i, v in enumerate(block):
                q[b * 32 + i] = max(-127, min(127, round_away(f32(v * inv))))
    return q, s


def quantize_inputs() -> np.ndarray:
    values = []
    for v in range(-126, 127):
        h = f32(v + 0.5)
        values += [f32(127), h, np.nextafter(h, f32(-np.inf)), np.nextafter(h, f32(np.inf))] + [f32(0)] * 28
    for amplitude in (0.0, 1.0, 1000.0, 1e-30, 1e-40):
        values += [f32((i % 32 - 16) * f32(amplitude)) for i in range(64)]
    for e in range(-149, -110, 3):  # blocks whose scale is subnormal or whose inverse overflows
        scale = f32(np.ldexp(1.0, e))
        values += [f32(((i * 7) % 15 - 7) * scale) for i in range(32)]
    for special in (0.0, -0.0, 1.4e-45, np.finfo(np.float32).max, np.nan, np.inf, -np.inf):
        values += [f32(special) if i == 17 else f32(0) for i in range(32)]
    return np.array(values, dtype=np.float32)


def q8_kat_case(frames: int, width: int, rows: int):
    idx = np.arange(frames * width)
    values = np.select([idx % 5 == 0, idx % 5 == 1, idx % 5 == 2, idx % 5 == 3],
                       [-1.0, 1.0, 0.0, -0.5], 0.1).astype(np.float32)
    w = np.array([-128, 127, 0, -127], dtype=np.int8)[np.arange(width * rows) % 4].reshape(rows, width)
    ws = np.where(np.arange(width * rows // 32) % 2 == 0, f32(0.013), f32(-0.007)).astype(np.float32)
    ws = ws.reshape(rows, width // 32)
    bias = (np.arange(rows) * f32(0.125)).astype(np.float32)
    q, xs = quantize_reference(values)
    q = q.reshape(frames, width).astype(np.int64)
    xs = xs.reshape(frames, width // 32)
    blocks = width // 32
    dots = np.einsum("tbk,rbk->trb", q.reshape(frames, blocks, 32), w.astype(np.int64).reshape(rows, blocks, 32))
    out = np.zeros((frames, rows), dtype=np.float32)
    for t in range(frames):
        for r in range(rows):
            acc = f32(0)
            for b in range(blocks):
                acc = f32(acc + f32(f32(f32(dots[t, r, b]) * ws[r, b]) * xs[t, b]))
            out[t, r] = f32(bias[r] + acc)
    return values, w, ws, bias, out


def main():
    x = quantize_inputs()
    q, s = quantize_reference(x)
    np.savez_compressed(os.path.join(HERE, "quantize_kat.npz"), input=x, q=q, scales=s)
    cases = {}
    for frames in (1, 3, 17):
        for width in (32, 96, 1024):
            for rows in (1, 3, 19, 32):
                v, w, ws, bias, out = q8_kat_case(frames, width, rows)
                cases[f"{frames}x{width}x{rows}"] = out
    np.savez_compressed(os.path.join(HERE, "q8_kat.npz"), **cases)
    print("wrote", len(cases), "Q8 cases and", x.size // 32, "quantize blocks")


if __name__ == "__main__":
    main()

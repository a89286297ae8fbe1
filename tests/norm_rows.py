"""Rows for the RMSNorm square-sum order tests (shared by the CPU and GPU
tests).

The reference sums a row's squares in double in four chains over x[4i + j]
(TensorMath.Elementwise.cs:58-71); the GPU kernels sum them as pairwise trees
and keep the tree's float mean only where no summation order can round to
another float. These rows make the two orders' float means differ."""
import numpy as np

f32 = np.float32


def crafted(width: int, rng) -> np.ndarray:
    """x[0] = 1 leads chain 0, whose other values are tiny: each square is
    just under half an ulp of the running sum, so the reference's chain drops
    every one of them, while a tree adds them among themselves first and
    keeps most of their total. x[1] and x[3] bring the sum just below the
    float rounding midpoint 1 + 2^-24 of width * mean, so the tree's extra
    lifts its mean one float above the reference's in a good share of these
    rows (the tests pick those with the oracle)."""
    x = np.zeros(width, f32)
    x[0] = 1.0
    x[4::4] = f32(rng.uniform(0.69, 0.705) * 2.0 ** -26)
    x[1] = f32(2.0 ** -12 * (1 - 2.0 ** -24))
    x[3] = f32(rng.uniform(0.0, 8.0) * 2.0 ** -26)
    perm = rng.permutation(width // 4)  # move the four chains' groups around
    return x.reshape(-1, 4)[perm].reshape(-1) if rng.random() < 0.5 else x


def midpoint(width: int) -> np.ndarray:
    """A square sum of exactly 1 + 2^-24: width * mean is a float rounding
    midpoint (ties to even), which no tree can settle."""
    x = np.zeros(width, f32)
    x[0] = 1.0
    x[width // 2 + 1] = f32(2.0 ** -12)
    return x


def inverse(mean, eps) -> np.float32:
    """1f / sqrt(mean + eps) in float32 (TensorMath.Elementwise.cs:78)."""
    return f32(1) / np.sqrt(f32(mean) + f32(eps))


def mismatching(oracle, width: int, count: int, seed: int, eps: float = 1e-6) -> np.ndarray:
    """`count` crafted rows, scaled by powers of two (which keeps every sum
    exact relative to the others), on which the tree order would give
    another RMSNorm inverse than the reference's order: their float means
    differ and the difference survives + eps, the square root and the
    reciprocal (checked with the oracle's restatements of both orders)."""
    rng = np.random.default_rng(seed)
    rows = []
    while len(rows) < count:
        x = crafted(width, rng) * f32(2.0 ** int(rng.integers(-6, 12)))
        tree, ref = oracle.sum_sq_gpu_tree(x), oracle.sum_sq_reference(x)
        if inverse(f32(tree / width), eps) != inverse(f32(ref / width), eps):
            rows.append(x)
    return np.stack(rows)

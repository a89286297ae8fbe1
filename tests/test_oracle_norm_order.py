"""RMSNorm square-sum order (TensorMath.Elementwise.cs:58-71).

The reference sums squares in double in four chains over x[4i + j], combined
(s0 + s2) + (s1 + s3). The GPU kernels sum them as pairwise trees and keep the
tree's float mean only when the orders' error bounds cannot straddle a float
rounding boundary (rms_mean in fah_device.h); otherwise they form the
reference's chains. Checked here on the CPU: the oracle's restatement of the
reference order against numpy's sequential sums, the restatement of the GPU
tree against an independent numpy tree, and over many rows (N(0,1), layer
activations captured from a decode, crafted rows) that the GPU's test never
settles on a mean other than the reference's. FAH_NORM_ROWS raises the row
counts (the design notes quote a run at 10^8 rows per case)."""
import os

import numpy as np
import pytest

from tests import norm_rows
from funasrnet_amd import model

f32, f64 = np.float32, np.float64


def chains_numpy(x):
    """The reference's chains with numpy's sequential cumulative sums."""
    sq = x.astype(f64) ** 2
    n4 = (x.size // 4) * 4
    s = [np.cumsum(sq[j:n4:4])[-1] if n4 else f64(0) for j in range(4)]
    r = (s[0] + s[2]) + (s[1] + s[3])
    for k in range(n4, x.size):
        r = r + sq[k]
    return r


def tree_numpy(x):
    """The GPU kernels' tree (width 128: two 64-channel trees; else 256
    threads of four values, 64-lane trees, wave sums in order)."""
    def pairwise(v):
        while v.size > 1:
            v = v[0::2] + v[1::2]
        return v[0]
    sq = x.astype(f64) ** 2
    if x.size == 128:
        return pairwise(sq[:64]) + pairwise(sq[64:])
    lanes = np.zeros(256)
    for c in range(4):
        for t in range(256):
            e = c * 1024 + 4 * t
            if e < x.size:
                lanes[t] = lanes[t] + (sq[e] + sq[e + 1])
                lanes[t] = lanes[t] + (sq[e + 2] + sq[e + 3])
    total = f64(0)
    for w in range(4):
        total = total + pairwise(lanes[64 * w:64 * w + 64])
    return total


@pytest.mark.parametrize("width", [128, 130, 1024])
def test_oracle_rms_norm_is_the_reference_order(oracle_lib, width):
    """oracle_rms_norm bit for bit against the chains restated with numpy,
    then 1f / sqrt((float)(S / width) + eps) and (x * inverse) * scale in
    float32 (each IEEE-rounded)."""
    rng = np.random.default_rng(width)
    eps = f32(1e-6)
    for scale_row in range(20):
        x = (rng.standard_normal(width) * np.exp(rng.standard_normal(width) * 2)).astype(f32)
        if scale_row % 5 == 0:
            x = norm_rows.crafted(width - width % 4, rng) if width % 4 == 0 else x
        scale = rng.standard_normal(width).astype(f32)
        s = chains_numpy(x)
        assert oracle_lib.sum_sq_reference(x) == s
        inverse = f32(1) / np.sqrt(f32(s / width) + eps)
        expected = (x * inverse) * scale
        got = oracle_lib.rms_norm(x, width, scale, float(eps))
        assert np.array_equal(got.view(np.uint32), expected.astype(f32).view(np.uint32))


@pytest.mark.parametrize("width", [128, 1024])
def test_gpu_tree_restatement(oracle_lib, width):
    rng = np.random.default_rng(7 + width)
    for _ in range(50):
        x = (rng.standard_normal(width) * np.exp(rng.standard_normal(width) * 3)).astype(f32)
        assert oracle_lib.sum_sq_gpu_tree(x) == tree_numpy(x)


def test_crafted_rows_differ_and_are_left_to_the_reference_order(oracle_lib):
    for width in (128, 1024):
        rows = norm_rows.mismatching(oracle_lib, width, 16, seed=width)
        for x in rows:
            tree, ref = oracle_lib.sum_sq_gpu_tree(x), oracle_lib.sum_sq_reference(x)
            assert f32(tree / width) != f32(ref / width)
            # The difference reaches the normalised row: the tree order would be visible.
            scale = np.ones(width, f32)
            tree_row = (x * norm_rows.inverse(f32(tree / width), 1e-6)) * scale
            assert not np.array_equal(tree_row, oracle_lib.rms_norm(x, width, scale, 1e-6))
            settled, _ = oracle_lib.rms_mean_settled(tree, width)
            assert not settled
        settled, _ = oracle_lib.rms_mean_settled(oracle_lib.sum_sq_gpu_tree(norm_rows.midpoint(width)), width)
        assert not settled
        for special in (np.inf, np.nan):
            # Infinite and NaN sums are such in any order: settled, same mean.
            x = np.ones(width, f32)
            x[3] = special
            settled, mean = oracle_lib.rms_mean_settled(oracle_lib.sum_sq_gpu_tree(x), width)
            ref = f32(oracle_lib.sum_sq_reference(x) / width)
            assert settled and (mean == ref or (np.isnan(mean) and np.isnan(ref)))
        tiny = np.zeros(width, f32)
        tiny[0] = f32(1e-40)  # square sum below 2^-126: the reference path
        assert not oracle_lib.rms_mean_settled(oracle_lib.sum_sq_gpu_tree(tiny), width)[0]
        assert not oracle_lib.rms_mean_settled(0.0, width)[0]  # all-zero rows take the reference path


@pytest.fixture(scope="module")
def activations(oracle_lib):
    """Input rows of every RMSNorm of a Qwen3-0.6B-shaped decode (synthetic
    weights, seed 0): 40 prefix rows and 4 greedy steps."""
    oracle_lib.set_threads(min(8, os.cpu_count() or 1))
    cfg = model.QWEN3_0_6B
    w = model.synthetic(cfg, seed=0)
    d = oracle_lib.Decoder(w, capacity=64)
    try:
        d.capture_norms(44 * 57, 44 * 28 * 24)
        logits = d.decode(np.random.default_rng(0).standard_normal((40, cfg.width)).astype(f32), 40)
        for _ in range(4):
            logits = d.decode(d.embed([oracle_lib.greedy(logits)]), 1)
        wide, head = d.captured()
        return wide.copy(), head.copy()
    finally:
        d.close()


def test_gpu_order_never_settles_on_another_mean(oracle_lib, activations):
    """Counts over sampled rows: the tree's own float mean against the
    reference's, how often the GPU's test leaves a row to the reference's
    chains, and that it never settles on a wrong mean."""
    rows = int(os.environ.get("FAH_NORM_ROWS", "200000"))
    wide, head = activations
    normal = np.random.default_rng(3).standard_normal(1 << 20).astype(f32)
    crafted = np.concatenate([norm_rows.crafted(1024, np.random.default_rng(s)) for s in range(64)])
    cases = [("N(0,1)", normal, 1024, False, rows), ("N(0,1)", normal, 128, False, 8 * rows),
             ("activations", wide, 1024, True, rows), ("activations", head, 128, True, 8 * rows),
             ("crafted", crafted, 1024, True, rows // 10)]
    for name, pool, width, rowwise, n in cases:
        total, differ, unsettled, wrong = oracle_lib.norm_order_stats(pool, width, n, 11, rowwise=rowwise)
        print(f"{name} width {width}: {total} rows, tree mean differs {differ}, "
              f"left to the reference order {unsettled}, settled wrongly {wrong}")
        assert wrong == 0
        assert unsettled >= differ
        if name != "crafted":
            assert unsettled <= max(20, total // 10000)
        else:
            assert differ > 0

"""fah_quantized_linear_noalloc (the allocation-free variant of
fah_quantized_linear, IQuantizedComputeBackend.TryQuantizedLinear) gives the
same output bits as fah_quantized_linear, on two calls in a row (the second
smaller, so stale workspace contents from the first would show), on both
the MFMA GEMM path (frames >= 4) and the GEMV path, and rejects a projection
larger than its fixed workspace."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _weight(rng, rows, cols):
    from funasrnet_amd.model import Q8Tensor
    q = rng.integers(-128, 128, size=(rows, cols), dtype=np.int8)
    s = (np.abs(rng.standard_normal((rows, cols // 32))) * 0.02 / 127).astype(np.float16).astype(np.float32)
    return Q8Tensor("w", q, s)


def _call(lib, name, backend, x, frames, w, bias, rows):
    from funasrnet_amd import hip
    out = np.full(frames * rows, np.nan, dtype=np.float32)
    fp = ctypes.POINTER(ctypes.c_float)
    b = None if bias is None else bias.ctypes.data_as(fp)
    rc = getattr(lib, name)(backend.handle, x.ctypes.data_as(fp), frames, w.handle, b, out.ctypes.data_as(fp))
    return rc, out


def test_noalloc_matches_quantized_linear():
    from funasrnet_amd import hip
    lib = hip.load()
    rng = np.random.default_rng(91)
    backend = hip.HipBackend(0)
    try:
        cases = [(17, 1024, 3072, False), (1, 1024, 2048, True)]  # the second call is smaller
        for frames, cols, rows, with_bias in cases:
            print(f"noalloc frames={frames} cols={cols} rows={rows} bias={with_bias}", flush=True)
            w = backend.weight(_weight(rng, rows, cols))
            x = rng.standard_normal(frames * cols).astype(np.float32)
            bias = rng.standard_normal(rows).astype(np.float32) if with_bias else None
            rc_a, ref = _call(lib, "fah_quantized_linear", backend, x, frames, w, bias, rows)
            rc_b, got = _call(lib, "fah_quantized_linear_noalloc", backend, x, frames, w, bias, rows)
            assert rc_a == rc_b == hip.OK, lib.fah_last_error()
            assert np.array_equal(ref.view(np.uint32), got.view(np.uint32))
        # Larger than the 8 MiB workspace: rejected, output untouched.
        frames, cols, rows = 128, 1024, 16384
        w = backend.weight(_weight(rng, rows, cols))
        x = rng.standard_normal(frames * cols).astype(np.float32)
        rc, out = _call(lib, "fah_quantized_linear_noalloc", backend, x, frames, w, None, rows)
        assert rc == hip.ERROR_ARGUMENT and b"workspace" in lib.fah_last_error()
        assert np.all(np.isnan(out))
    finally:
        backend.close()

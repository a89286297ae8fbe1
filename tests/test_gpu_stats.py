"""Seam-call statistics (fah_context_statistics) and the per-call observer:
the counters VulkanFloatBackend.Statistics() keeps (calls per kind, declined
calls, bytes each way, end-to-end time; VulkanFloatBackend.cs:86-118) plus
device time, and a LinearMeasured-style callback per call
(TensorMath.cs:37-40, 198)."""
import numpy as np
import pytest

from funasrnet_amd import model

pytestmark = pytest.mark.gpu


def test_statistics_and_observer():
    from funasrnet_amd.hip import HipBackend
    from funasrnet_amd.model import Q8Tensor
    b = HipBackend(0)  # default minimum of 250000 multiply-adds
    try:
        rng = np.random.default_rng(3)
        q = rng.integers(-127, 128, size=(2048, 1024), dtype=np.int8)
        s = (np.abs(rng.standard_normal((2048, 32))) * 1e-4).astype(np.float16).astype(np.float32)
        w = Q8Tensor("w", q, s)
        small = Q8Tensor("s", q[:8, :64].copy(), s[:8, :2].copy())
        f = (rng.random((512, 1024)) - 0.5).astype(np.float32)
        seen = []
        b.set_call_observer(lambda *args: seen.append(args))
        print("seam statistics: 3 Q8 calls, 1 declined, 1 group, 1 FP32", flush=True)
        for frames in (1, 2, 5):
            x = rng.standard_normal((frames, 1024)).astype(np.float32)
            out = np.empty(frames * 2048, np.float32)
            assert b.try_quantized_linear(x, frames, w, None, out)
        out = np.full(8, 7.0, np.float32)
        assert not b.try_quantized_linear(rng.standard_normal(64).astype(np.float32), 1, small, None, out)
        assert np.all(out == 7.0)
        x = rng.standard_normal((4, 1024)).astype(np.float32)
        assert b.try_linear_many(x, 4, [w, w]) is not None
        y = np.empty(4 * 512, np.float32)
        assert b.try_linear(x, 4, f, None, y)
        st = b.statistics()
        ql = st["quantized_linear"]
        assert ql["calls"] == 3 and ql["declined"] == 1
        assert ql["operations"] == 8 * 1024 * 2048
        assert ql["uploaded_bytes"] == 8 * 1024 * 4 and ql["downloaded_bytes"] == 8 * 2048 * 4
        assert 0 < ql["device_ms"] <= ql["total_ms"]
        assert st["linear_many"]["calls"] == 1 and st["linear_many"]["operations"] == 4 * 1024 * 4096
        assert st["linear"]["calls"] == 1 and st["linear"]["downloaded_bytes"] == 4 * 512 * 4
        assert st["attention"]["calls"] == 0
        assert [a[:4] for a in seen] == [("quantized_linear", 1, 1024, 2048), ("quantized_linear", 2, 1024, 2048),
                                         ("quantized_linear", 5, 1024, 2048), ("linear_many", 4, 1024, 4096),
                                         ("linear", 4, 1024, 512)]
        assert all(0 < a[4] <= a[5] for a in seen)
        b.set_call_observer(None)
        b.reset_statistics()
        assert all(v == 0 for rec in b.statistics().values() for v in rec.values())
        out = np.empty(2048, np.float32)
        assert b.try_quantized_linear(rng.standard_normal(1024).astype(np.float32), 1, w, None, out)
        assert len(seen) == 5 and b.statistics()["quantized_linear"]["calls"] == 1
    finally:
        b.close()

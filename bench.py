"""Benchmark: Qwen3-0.6B Q8_0 batch-1 greedy decode on one MI355X.

Workload (the decode configuration the metric is quoted on): the synthetic
Qwen3-0.6B-shaped decoder (28 layers, hidden 1024, 16/8 heads x 128,
FFN 3072, vocab 151936 tied, Q8_0 int8 U{-127..127}, fp16 scales
|N(0,0.02)|/127, seed 0), a 150-row N(0,1) embedding prefix, then greedy
decode steps with the F16 KV cache. A step is one decoded token: the whole
decoder on the device (embedding of the previous greedy token, 28 layers,
final norm, tied lm_head, argmax) -- one launch of the persistent
decode_step_kernel (or one captured HIP graph of the multi-kernel path with
FAH_PERSISTENT=0).

Printed: one JSON line with decode tok/s; the roofline of the dominant
kernel (the decode step: algorithmic bytes per token -- Q8_0 weights, K/V
reads, norm weights -- over the average launch time, HIP events on the
context stream); the lm_head-shape Q8_0 GEMV (1024->151936, four rotated
weight copies so every launch streams from HBM); and the CPU oracle timed on
this host on repeated 128-step passes of the same decode (about 10 s).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
PREFIX = 150


def gemv_roofline(backend, weights, repeats: int = 40):
    """Average duration of the Q8_0 GEMV kernel at the lm_head shape."""
    from funasrnet_amd import device
    from funasrnet_amd.model import Q8Tensor

    lm = weights.lm_head
    copies = [backend.weight(Q8Tensor(f"lm{i}", lm.quantized, lm.scales)) for i in range(4)]
    rows, cols = lm.rows, lm.columns
    rng = np.random.default_rng(7)
    x = rng.standard_normal(cols).astype(np.float32)
    xd = device.DeviceArray.from_numpy(x)
    q = device.DeviceArray(cols, np.int8)
    s = device.DeviceArray(cols // 32, np.float32)
    out = device.DeviceArray(rows, np.float32)
    backend.quantize_device(xd.ptr, cols, q.ptr, s.ptr)
    for i in range(8):
        backend.gemv_device(q.ptr, s.ptr, 1, copies[i % 4], out.ptr)
    backend.synchronize()
    start, end = device.Event(), device.Event()
    start.record(backend.stream)
    for i in range(repeats):
        backend.gemv_device(q.ptr, s.ptr, 1, copies[i % 4], out.ptr)
    end.record(backend.stream)
    end.synchronize()
    avg_us = start.elapsed_ms(end) * 1000.0 / repeats
    algorithmic = rows * cols * 34 // 32 + cols + 4 * (cols // 32) + 4 * rows
    device_bytes = copies[0].device_bytes
    for c in copies:
        c.close()
    return {
        "kernel": "q8_gemv_kernel (Q8_0 GEMV, 1024->151936)",
        "avg_us": avg_us,
        "algorithmic_bytes": algorithmic,
        "device_bytes": device_bytes,
        "achieved_gbs": algorithmic / (avg_us * 1e-6) / 1e9,
    }


GEMV_SHAPES = [(1024, 2048), (1024, 1024), (2048, 1024), (1024, 3072), (3072, 1024), (1024, 151936)]
MFMA_PEAK_INT8_OPS = 5.0e15


def gemv_sweep(backend, rotate_bytes: int = 512 << 20):
    """Q8_0 GEMV at the decoder's projection shapes (K -> N), each launch on
    a different copy of the weight, rotating through at least `rotate_bytes`
    so that launches stream from HBM rather than the 256 MB MALL."""
    from funasrnet_amd import device
    from funasrnet_amd.model import Q8Tensor

    rng = np.random.default_rng(3)
    results = []
    for K, N in GEMV_SHAPES:
        q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
        sc = (np.abs(rng.standard_normal((N, K // 32))) * 0.02 / 127).astype(np.float16).astype(np.float32)
        tensor = Q8Tensor("sweep", q, sc)
        algorithmic = N * K * 34 // 32 + K + 4 * (K // 32) + 4 * N
        copies = [backend.weight(tensor) for _ in range(max(2, -(-rotate_bytes // algorithmic)))]
        x = rng.standard_normal(K).astype(np.float32)
        xd = device.DeviceArray.from_numpy(x)
        xq = device.DeviceArray(K, np.int8)
        xs = device.DeviceArray(K // 32, np.float32)
        out = device.DeviceArray(N, np.float32)
        backend.quantize_device(xd.ptr, K, xq.ptr, xs.ptr)
        for c in copies:
            backend.gemv_device(xq.ptr, xs.ptr, 1, c, out.ptr)
        backend.synchronize()
        start, end = device.Event(), device.Event()
        start.record(backend.stream)
        for c in copies:
            backend.gemv_device(xq.ptr, xs.ptr, 1, c, out.ptr)
        end.record(backend.stream)
        end.synchronize()
        avg_us = start.elapsed_ms(end) * 1000.0 / len(copies)
        gbs = algorithmic / (avg_us * 1e-6) / 1e9
        results.append({"shape": f"{K}->{N}", "avg_us": round(avg_us, 3), "algorithmic_bytes": algorithmic,
                        "achieved_gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "copies": len(copies)})
        for c in copies:
            c.close()
        for arr in (xd, xq, xs, out):
            arr.free()
    return results


FP32_MFMA_PEAK = 157.3e12


def float_gemv_sweep(backend, rotate_bytes: int = 512 << 20):
    """FP32 ("original weights") GEMV at the decoder's projection shapes
    (K -> N, 4 B per weight), each launch on a different copy, rotating
    through at least `rotate_bytes` so that launches stream from HBM."""
    from funasrnet_amd import device

    rng = np.random.default_rng(5)
    results = []
    for K, N in GEMV_SHAPES:
        w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        algorithmic = 4 * (N * K + K + N)
        copies = [backend.float_weight(w.copy()) for _ in range(max(2, -(-rotate_bytes // algorithmic)))]
        x = device.DeviceArray.from_numpy(rng.standard_normal(K).astype(np.float32))
        out = device.DeviceArray(N, np.float32)
        for c in copies:
            backend.linear_device(x.ptr, 1, c, None, out.ptr)
        backend.synchronize()
        start, end = device.Event(), device.Event()
        start.record(backend.stream)
        for c in copies:
            backend.linear_device(x.ptr, 1, c, None, out.ptr)
        end.record(backend.stream)
        end.synchronize()
        avg_us = start.elapsed_ms(end) * 1000.0 / len(copies)
        gbs = algorithmic / (avg_us * 1e-6) / 1e9
        results.append({"shape": f"{K}->{N}", "avg_us": round(avg_us, 3), "algorithmic_bytes": algorithmic,
                        "achieved_gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "copies": len(copies)})
        for c in copies:
            c.close()
        backend._weights.clear()
        x.free()
        out.free()
    return results


def encoder_float(backend, frames: int = 1000, repeats: int = 20):
    """The encoder's FP32 operations at one 60 s segment's shape (1000
    frames, width 512, 4 heads; FunEncoder.cs:100-300): the projections on
    fp32 MFMA (TFLOP/s against the 157.3 TFLOP/s dense fp32 peak) and the
    non-causal attention, device-resident, HIP events over `repeats` runs."""
    from funasrnet_amd import device

    rng = np.random.default_rng(6)
    out = {"frames": frames, "linear": []}
    for K, N in ((512, 1536), (512, 512), (512, 2048), (2048, 512)):
        w = backend.float_weight((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
        x = device.DeviceArray.from_numpy(rng.standard_normal((frames, K)).astype(np.float32))
        y = device.DeviceArray(frames * N, np.float32)
        backend.linear_device(x.ptr, frames, w, None, y.ptr)
        backend.synchronize()
        start, end = device.Event(), device.Event()
        start.record(backend.stream)
        for _ in range(repeats):
            backend.linear_device(x.ptr, frames, w, None, y.ptr)
        end.record(backend.stream)
        end.synchronize()
        us = start.elapsed_ms(end) * 1000.0 / repeats
        flops = 2.0 * frames * N * K
        out["linear"].append({"shape": f"{frames}x{K}->{N}", "avg_us": round(us, 2),
                              "tflops": round(flops / (us * 1e-6) / 1e12, 2),
                              "frac_of_fp32_mfma_peak": round(flops / (us * 1e-6) / FP32_MFMA_PEAK, 4)})
        x.free()
        y.free()
    backend._weights.clear()
    width, heads = 512, 4
    q, k, v = (device.DeviceArray.from_numpy(rng.standard_normal((frames, width)).astype(np.float32)) for _ in range(3))
    y = device.DeviceArray(frames * width, np.float32)
    backend.attention_device(q.ptr, k.ptr, v.ptr, frames, width, heads, y.ptr)
    backend.synchronize()
    start, end = device.Event(), device.Event()
    start.record(backend.stream)
    for _ in range(repeats):
        backend.attention_device(q.ptr, k.ptr, v.ptr, frames, width, heads, y.ptr)
    end.record(backend.stream)
    end.synchronize()
    us = start.elapsed_ms(end) * 1000.0 / repeats
    flops = 4.0 * frames * frames * width
    out["attention"] = {"shape": f"{frames} frames x {width} ({heads} heads)", "avg_us": round(us, 2),
                        "tflops": round(flops / (us * 1e-6) / 1e12, 2)}
    for a in (q, k, v, y):
        a.free()
    return out


def prefill_ttft(backend, weights, rows_list=(375, 750)):
    """Time to first token: one decode call on `rows` N(0,1) rows from
    position 0 (the MFMA GEMM prefill) plus the greedy pick, wall clock, best
    of three. The call copies the rows in (rows x 4 KiB) and the logits out
    (0.6 MB) over PCIe; both are inside the time."""
    from funasrnet_amd import device
    from funasrnet_amd.hip import HipDecoder

    cfg = weights.config
    qw, kvw = cfg.heads * cfg.head_size, cfg.kv_heads * cfg.head_size
    per_row = 2 * cfg.layers * (cfg.width * (qw + 2 * kvw) + qw * cfg.width + 3 * cfg.width * cfg.ffn)
    dec = HipDecoder(backend, weights, capacity=max(rows_list) + 8)
    out = []
    try:
        for rows in rows_list:
            x = np.random.default_rng(rows).standard_normal((rows, cfg.width)).astype(np.float32)
            dec.reset()
            dec.decode(x, rows)
            best = None
            for _ in range(3):
                dec.reset()
                device.synchronize()
                t0 = time.perf_counter()
                dec.decode(x, rows)
                dec.greedy()
                ms = (time.perf_counter() - t0) * 1e3
                best = ms if best is None else min(best, ms)
            ops = per_row * rows + 2 * cfg.vocab * cfg.width
            out.append({"rows": rows, "ttft_ms": round(best, 3), "int8_ops": int(ops),
                        "achieved_tops": round(ops / (best * 1e-3) / 1e12, 2),
                        "frac_of_int8_mfma_peak": round(ops / (best * 1e-3) / MFMA_PEAK_INT8_OPS, 5)})
    finally:
        dec.close()
    return out


def long_kv(backend, weights, positions: int = 4096, steps: int = 64):
    """Decode with a long cache: K/V rows [0, positions) pre-filled with
    fp16(N(0,1)) in every layer, one row decoded at `positions`, then `steps`
    timed greedy steps. Algorithmic bytes per token include the K/V reads."""
    from funasrnet_amd import device
    from funasrnet_amd.hip import HipDecoder

    cfg = weights.config
    dec = HipDecoder(backend, weights, capacity=positions + steps + 64)
    try:
        rng = np.random.default_rng(4)
        width = cfg.kv_heads * cfg.head_size
        for layer in range(cfg.layers):
            k = rng.standard_normal((positions, width)).astype(np.float16)
            v = rng.standard_normal((positions, width)).astype(np.float16)
            dec.kv_write(layer, k, v)
        dec.set_position(positions)
        dec.decode(rng.standard_normal((1, cfg.width)).astype(np.float32), 1)
        device.synchronize()
        start, end = device.Event(), device.Event()
        start.record(backend.stream)
        dec.generate(steps)
        end.record(backend.stream)
        end.synchronize()
        ms = start.elapsed_ms(end) / steps
        kv = sum(114688 * (positions + 1 + i + 1) for i in range(steps)) / steps
        step_bytes = cfg.weight_bytes_per_token() + kv
        gbs = step_bytes / (ms * 1e-3) / 1e9
        out = {"positions": positions, "steps": steps, "ms_per_step": round(ms, 4), "tok_s": round(1000.0 / ms, 2),
               "bytes_per_token": int(step_bytes), "achieved_gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
    finally:
        dec.close()
    out["attention"] = long_kv_attention(backend, weights, positions)
    out["shorter_caches"] = {str(p): long_kv_tok_s(backend, weights, p) for p in (750, 2048)}
    return out


def long_kv_tok_s(backend, weights, positions: int, steps: int = 32) -> float:
    """Greedy decode tok/s after `positions` cached fp16(N(0,1)) rows (the
    persistent kernel's long-cache attention below its switch)."""
    from funasrnet_amd import device
    from funasrnet_amd.hip import HipDecoder

    cfg = weights.config
    dec = HipDecoder(backend, weights, capacity=positions + steps + 64)
    try:
        rng = np.random.default_rng(4)
        for layer in range(cfg.layers):
            dec.kv_write(layer, rng.standard_normal((positions, cfg.kv_width)).astype(np.float16),
                         rng.standard_normal((positions, cfg.kv_width)).astype(np.float16))
        dec.set_position(positions)
        dec.decode(rng.standard_normal((1, cfg.width)).astype(np.float32), 1)
        dec.generate(4)
        device.synchronize()
        start, end = device.Event(), device.Event()
        start.record(backend.stream)
        dec.generate(steps)
        end.record(backend.stream)
        end.synchronize()
        return round(1000.0 * steps / start.elapsed_ms(end), 2)
    finally:
        dec.close()


def long_kv_attention(backend, weights, positions: int, steps: int = 16):
    """The attention alone at a long cache, K/V-read GB/s = the K/V bytes of
    a layer over its attention time. The decoder is created with
    FAH_TIMELINE=1 and FAH_ATTENTION_TIMES=1 and runs the steps one by one.

    Steps on the multi-kernel path (past the persistent kernel's range):
    HIP events around every layer's attention launches. Steps on the
    persistent kernel: each layer's attention time from the phase timeline,
    from the attention workgroups' q/k/v hand-over (the projection
    workgroups then start reading the K rows for the scores) to the
    publication of the attention output, median over the 16 attention
    workgroups, layers 1..L-2 and steps."""
    from funasrnet_amd.hip import HipDecoder

    cfg = weights.config
    keys = ("FAH_TIMELINE", "FAH_ATTENTION_TIMES")
    old = {k: os.environ.get(k) for k in keys}
    os.environ.update({k: "1" for k in keys})
    try:
        dec = HipDecoder(backend, weights, capacity=positions + steps + 64)
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v
    try:
        rng = np.random.default_rng(4)
        width = cfg.kv_heads * cfg.head_size
        for layer in range(cfg.layers):
            k = rng.standard_normal((positions, width)).astype(np.float16)
            v = rng.standard_normal((positions, width)).astype(np.float16)
            dec.kv_write(layer, k, v)
        dec.set_position(positions)
        dec.decode(rng.standard_normal((1, cfg.width)).astype(np.float32), 1)
        dec.attention_time()
        spans = []
        for i in range(steps):
            dec.generate(1)
            tl = dec.timeline()
            if tl is not None:
                tl = tl.astype(np.int64)[:cfg.heads]
                for layer in range(1, cfg.layers - 1):
                    e = 16 * layer + 1
                    spans.append(float(np.median(tl[:, e + 7] - tl[:, e + 0])) * 0.01)  # 100 MHz ticks -> us
        ms, counted = dec.attention_time()
        if counted == 0:
            us = float(np.median(spans))
            n = positions + 1 + steps // 2
            kv_layer = 114688 // cfg.layers * n
            gbs = kv_layer / (us * 1e-6) / 1e9
            return {"kernels": "decode_step_kernel attention (phase timeline)", "steps": steps,
                    "us_per_layer": round(us, 2), "kv_bytes_per_layer": int(kv_layer), "kv_read_gbs": round(gbs, 1),
                    "frac": round(gbs / HBM_PEAK_GBS, 4)}
        kv = sum(114688 * (positions + 1 + i + 1) for i in range(counted))
        us_per_layer = ms * 1000.0 / counted / cfg.layers
        gbs = kv / (ms * 1e-3) / 1e9
        return {"kernels": "attn_scores_kernel + attn_values_kernel", "steps": counted,
                "ms_per_token": round(ms / counted, 4), "us_per_layer": round(us_per_layer, 2),
                "kv_bytes_per_token": int(kv / counted), "kv_read_gbs": round(gbs, 1),
                "frac": round(gbs / HBM_PEAK_GBS, 4)}
    finally:
        dec.close()


def sessions_decode(backend, weights, count: int = 16, steps: int = 128, prefix: int = 150, warmup: int = 4,
                    check: int | None = None):
    """Lock-step decode of `count` sessions over one weight set: 150-row
    N(0,1) prefixes (seeds 1..count), `warmup` lock-step steps (the first
    call captures the step), then `steps` timed steps (wall clock around one
    call). Algorithmic bytes per step: the weights once plus every session's
    K/V rows."""
    from funasrnet_amd.hip import HipDecoder

    cfg = weights.config
    capacity = prefix + warmup + steps + 8
    parent = HipDecoder(backend, weights, capacity=capacity)
    sessions = [parent] + [parent.session() for _ in range(count - 1)]
    try:
        for seed, d in enumerate(sessions, 1):
            x = np.random.default_rng(seed).standard_normal((prefix, cfg.width)).astype(np.float32)
            d.decode(x, prefix)
        warm = HipDecoder.generate_sessions(sessions, warmup)
        t0 = time.perf_counter()
        toks = HipDecoder.generate_sessions(sessions, steps)
        wall = time.perf_counter() - t0
        ms = wall * 1e3 / steps
        start = prefix + warmup
        kv = count * sum(114688 * (start + i + 1) for i in range(steps)) / steps
        step_bytes = cfg.weight_bytes_per_token() + kv
        gbs = step_bytes / (ms * 1e-3) / 1e9
        distinct = len({tuple(t) for t in toks.tolist()})
        # The weight bytes one-token-at-a-time decoders would stream for the
        # same tokens, per second: count x the weights per step.
        effective = count * cfg.weight_bytes_per_token() / (ms * 1e-3) / 1e9
        result = {"sessions": count, "steps": steps, "ms_per_step": round(ms, 4),
                  "tok_s": round(count * 1000.0 / ms, 1), "bytes_per_step": int(step_bytes),
                  "achieved_gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                  "effective_weight_gbs": round(effective, 1), "distinct_token_rows": distinct}
    finally:
        for d in sessions[1:]:
            d.close()
        parent.close()
    if check is not None:
        result["oracle_check"] = sessions_oracle_check(weights, warm, toks, prefix, check)
    return result


def compare_sessions(got, expected):
    """Per-session token equality against the oracle's token lists (each
    session decoded alone), with the first differing step of each session
    that differs."""
    equal, first_divergence = 0, {}
    for i, (g, e) in enumerate(zip(got, expected)):
        e = e[: len(g)]
        if g == e:
            equal += 1
        else:
            first_divergence[i] = next((j for j, (a, b) in enumerate(zip(g, e)) if a != b), min(len(g), len(e)))
    return {"sessions_equal": equal, "sessions": len(got), "steps_compared": min(len(g) for g in got),
            "first_divergence": first_divergence}


def step_batcher_decode(backend, weights, count: int = 16, steps: int = 128, prefix: int = 150, expected=None):
    """Server-style decode: `count` worker threads, each with its own session
    and 150-row prefix (seeds 1..count), each calling the cross-context step
    batcher once per token (FunAsr.Transcribe's loop run by a pool's
    workers); aggregate tok/s over the threads' decode phase (wall clock),
    and the mean batch the batcher formed. With `expected` (the oracle's
    tokens of each session decoded alone) every session's tokens are
    compared with it."""
    import threading
    from funasrnet_amd.hip import HipDecoder, HipStepBatcher

    cfg = weights.config
    capacity = prefix + steps + 8
    parent = HipDecoder(backend, weights, capacity=capacity)
    sessions = [parent] + [parent.session() for _ in range(count - 1)]
    batcher = HipStepBatcher(parent, max_positions=capacity, window_us=2000)
    start_gate = threading.Barrier(count + 1)
    times = [0.0] * count
    errors = []
    got = [[] for _ in range(count)]

    def worker(i):
        try:
            d = sessions[i]
            d.decode(np.random.default_rng(i + 1).standard_normal((prefix, cfg.width)).astype(np.float32), prefix)
            batcher.join(d)
            start_gate.wait()
            for _ in range(steps):
                got[i].append(batcher.step(d))
            times[i] = time.perf_counter()
            batcher.leave(d)
        except Exception as e:  # reported in the result
            errors.append(repr(e))
            try:
                start_gate.abort()
            except Exception:
                pass

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(count)]
    try:
        for t in threads:
            t.start()
        start_gate.wait()
        t0 = time.perf_counter()
        for t in threads:
            t.join()
        wall = max(times) - t0
        batches, rows = batcher.stats()
        python = {"tok_s": round(count * steps / wall, 1), "ms_per_batch": round(wall * 1e3 / max(batches, 1), 4),
                  "batches": batches, "mean_batch": round(rows / max(batches, 1), 2), "errors": errors}
        if expected is not None:
            python["oracle_check"] = compare_sessions(got, expected)
    finally:
        batcher.close()
        for d in sessions[1:]:
            d.close()
        parent.close()
    native = step_batcher_native(backend, weights, count, steps, prefix, expected)
    # The native worker threads are the reference's kind of caller (a pool's
    # .NET threads); the Python threads' figure includes the interpreter lock.
    result = {"sessions": count, "steps": steps, "workers": "native threads", **native,
              "python_threads": python}
    return result


def step_batcher_native(backend, weights, count: int, steps: int, prefix: int, expected=None):
    """The same sessions and steps as step_batcher_decode, each session's
    steps issued by a native thread of funasrnet_amd/libfah_bench_workers.so
    (fah_bench_batcher_threads) through fah_batcher_step."""
    import ctypes
    from funasrnet_amd import build as fab
    from funasrnet_amd.hip import HipDecoder, HipStepBatcher, load

    workers = ctypes.CDLL(fab.BENCH_WORKERS)
    workers.fah_bench_batcher_threads.restype = ctypes.c_int
    workers.fah_bench_batcher_threads.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p),
                                                  ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_int32),
                                                  ctypes.POINTER(ctypes.c_double)]
    cfg = weights.config
    capacity = prefix + steps + 8
    parent = HipDecoder(backend, weights, capacity=capacity)
    sessions = [parent] + [parent.session() for _ in range(count - 1)]
    batcher = HipStepBatcher(parent, max_positions=capacity, window_us=2000)
    try:
        for i, d in enumerate(sessions):
            d.decode(np.random.default_rng(i + 1).standard_normal((prefix, cfg.width)).astype(np.float32), prefix)
            batcher.join(d)
        handles = (ctypes.c_void_p * count)(*[ctypes.cast(d.handle, ctypes.c_void_p).value for d in sessions])
        tokens = np.zeros((count, steps), dtype=np.int32)
        seconds = ctypes.c_double(0.0)
        step_fn = ctypes.cast(load().fah_batcher_step, ctypes.c_void_p)
        rc = workers.fah_bench_batcher_threads(step_fn, ctypes.cast(batcher.handle, ctypes.c_void_p), handles, count, steps,
                                               tokens.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), ctypes.byref(seconds))
        batches, rows = batcher.stats()
        wall = max(seconds.value, 1e-9)
        result = {"tok_s": round(count * steps / wall, 1), "ms_per_batch": round(wall * 1e3 / max(batches, 1), 4),
                  "batches": batches, "mean_batch": round(rows / max(batches, 1), 2),
                  "errors": [] if rc == 0 else [f"fah_batcher_step returned {rc}"]}
        if expected is not None:
            result["oracle_check"] = compare_sessions([list(t) for t in tokens.tolist()], expected)
        for d in sessions:
            batcher.leave(d)
        return result
    finally:
        batcher.close()
        for d in sessions[1:]:
            d.close()
        parent.close()


def sessions_oracle_check(weights, warm, toks, prefix: int, threads: int):
    """Every session's tokens (warm-up and timed steps) against the oracle
    decoding that session alone (FunAsr.Transcribe's loop, FunAsr.cs:167-178);
    the oracle's time doubles as the CPU baseline of the same workload."""
    import oracle

    used = oracle.set_threads(threads)
    cfg = weights.config
    count, steps = toks.shape[0], warm.shape[1] + toks.shape[1]
    equal, first_divergence, seconds, tokens = 0, {}, 0.0, []
    for i in range(count):
        x = np.random.default_rng(i + 1).standard_normal((prefix, cfg.width)).astype(np.float32)
        dec = oracle.Decoder(weights, capacity=prefix + steps + 8)
        try:
            logits = dec.decode(x, prefix)
            expected = []
            t0 = time.perf_counter()
            for _ in range(steps):
                t = oracle.greedy(logits)
                expected.append(t)
                logits = dec.decode(dec.embed([t]), 1)
            seconds += time.perf_counter() - t0
        finally:
            dec.close()
        tokens.append(expected)
        got = warm[i].tolist() + toks[i].tolist()
        if got == expected:
            equal += 1
        else:
            first_divergence[i] = next(j for j, (a, b) in enumerate(zip(got, expected)) if a != b)
    return {"sessions_equal": equal, "sessions": count, "steps_compared": steps,
            "first_divergence": first_divergence, "_tokens": tokens,
            "cpu": {"kind": "port", "cores": used, "tok_s": round(count * steps / seconds, 2),
                    "sample": f"oracle, each of the {count} sessions decoded alone for {steps} greedy steps "
                              f"after its {prefix}-row prefix (decode time only)"}}


def cpu_baseline(weights, prefix, tokens: int, threads: int, seconds_target: float):
    """The oracle (C restatement of the reference x64 path) on this host.

    Prefill once, then repeat the `tokens`-step greedy decode from the same
    post-prefill state (position rewound; the K/V rows it writes are written
    again identically) until about `seconds_target` seconds of decode ran.
    """
    import oracle

    used = oracle.set_threads(threads)
    dec = oracle.Decoder(weights, capacity=PREFIX + tokens + 8)
    try:
        first = dec.decode(prefix, prefix.shape[0])
        steps = 0
        passes = 0
        seconds = 0.0
        while passes == 0 or seconds < seconds_target:
            dec.set_position(PREFIX)
            logits = first
            t0 = time.perf_counter()
            for _ in range(tokens):
                t = oracle.greedy(logits)
                logits = dec.decode(dec.embed([t]), 1)
            seconds += time.perf_counter() - t0
            steps += tokens
            passes += 1
    finally:
        dec.close()
    return steps / seconds, used, seconds, passes


def host_cpu():
    """Model name, SIMD flags relevant to the Q8_0 path, and core counts of
    this host (from /proc/cpuinfo and the scheduler's affinity mask)."""
    model_name, flags, cores = "unknown", set(), set()
    phys = core = None
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                key, _, value = line.partition(":")
                key, value = key.strip(), value.strip()
                if key == "model name":
                    model_name = value
                elif key == "flags":
                    flags = set(value.split())
                elif key == "physical id":
                    phys = value
                elif key == "core id":
                    core = value
                elif not key and phys is not None:
                    cores.add((phys, core))
                    phys = core = None
            if phys is not None:
                cores.add((phys, core))
    except OSError:
        pass
    simd = [f for f in ("avx2", "fma", "avx_vnni", "avx512f", "avx512bw", "avx512_vnni", "amx_int8") if f in flags]
    available = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return {"model": model_name, "simd": simd, "physical_cores": len(cores) or None, "available_cpus": available}


def cpu_extra_baselines(weights, threads: int):
    """The oracle on this host beside each extra measurement, on bounded
    samples of the same workloads (each a few seconds)."""
    import oracle

    used = oracle.set_threads(threads)
    cfg = weights.config
    out = {}
    # GEMV sweep: the same shapes and generator; the small matrices stay in
    # the host caches across repetitions (no rotation on the CPU side).
    rng = np.random.default_rng(3)
    rows = []
    for K, N in GEMV_SHAPES:
        q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
        sc = (np.abs(rng.standard_normal((N, K // 32))) * 0.02 / 127).astype(np.float16).astype(np.float32)
        xq, xs = oracle.quantize(rng.standard_normal(K).astype(np.float32))
        algorithmic = N * K * 34 // 32 + K + 4 * (K // 32) + 4 * N
        reps, t0 = 0, time.perf_counter()
        while reps == 0 or time.perf_counter() - t0 < 0.3:
            oracle.gemv_quantized(xq, xs, q, sc)
            reps += 1
        us = (time.perf_counter() - t0) * 1e6 / reps
        rows.append({"shape": f"{K}->{N}", "avg_us": round(us, 1), "achieved_gbs": round(algorithmic / (us * 1e-6) / 1e9, 1)})
    out["gemv_sweep"] = {"kind": "port", "cores": used, "shapes": rows,
                         "sample": "oracle_q8_gemv_quantized, >=0.3 s of repetitions per shape"}
    # Prefill: one decode of the same N(0,1) rows from position 0 (+ greedy).
    pre = []
    for n in (375, 750):
        x = np.random.default_rng(n).standard_normal((n, cfg.width)).astype(np.float32)
        dec = oracle.Decoder(weights, capacity=n + 8)
        try:
            t0 = time.perf_counter()
            oracle.greedy(dec.decode(x, n))
            pre.append({"rows": n, "ttft_ms": round((time.perf_counter() - t0) * 1e3, 1)})
        finally:
            dec.close()
    out["prefill"] = {"kind": "port", "cores": used, "rows": pre, "sample": "one prefill per size"}
    # Long cache: 4,096 fp16 N(0,1) positions in every layer, 4 greedy steps.
    positions, steps = 4096, 4
    dec = oracle.Decoder(weights, capacity=positions + steps + 64)
    try:
        r = np.random.default_rng(4)
        width = cfg.kv_heads * cfg.head_size
        for layer in range(cfg.layers):
            k = r.standard_normal((positions, width)).astype(np.float16).astype(np.float32)
            v = r.standard_normal((positions, width)).astype(np.float16).astype(np.float32)
            dec.set_kv(layer, k, v)
        dec.set_position(positions)
        logits = dec.decode(r.standard_normal((1, cfg.width)).astype(np.float32), 1)
        t0 = time.perf_counter()
        for _ in range(steps):
            logits = dec.decode(dec.embed([oracle.greedy(logits)]), 1)
        sec = time.perf_counter() - t0
    finally:
        dec.close()
    out["long_kv"] = {"kind": "port", "cores": used, "tok_s": round(steps / sec, 2),
                      "sample": f"{steps} greedy steps after 4096 cached positions"}
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--cpu-tokens", type=int, default=128, help="decode steps per CPU pass")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU sample length")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the GEMV sweep, prefill, long-cache and sessions measurements")
    ap.add_argument("--extra-only", choices=["gemv_sweep", "prefill", "long_kv", "sessions", "float_gemv_sweep",
                                             "encoder_float", "step_batcher", "sessions_by_count"],
                    help="run one of the extra measurements alone and print its JSON (for profilers)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the batch-1 decode path runs on a single MI355X "
              f"(requested --gpus {args.gpus}); lock-step sessions would shard by giving each GPU its own "
              f"sessions and a copy of the weights.", file=sys.stderr)
        return 2
    if PREFIX + max(args.steps, args.warmup) + 1 > 2048:
        print("steps + prefix exceed the decoder capacity (2048)", file=sys.stderr)
        return 2

    from funasrnet_amd import device, model
    from funasrnet_amd.hip import HipBackend, HipDecoder

    cfg = model.QWEN3_0_6B
    weights = model.synthetic(cfg, seed=0)
    if args.extra_only:
        backend = HipBackend(0)
        run = {"gemv_sweep": lambda: gemv_sweep(backend), "prefill": lambda: prefill_ttft(backend, weights),
               "long_kv": lambda: long_kv(backend, weights), "sessions": lambda: sessions_decode(backend, weights),
               "float_gemv_sweep": lambda: float_gemv_sweep(backend), "encoder_float": lambda: encoder_float(backend),
               "step_batcher": lambda: step_batcher_decode(backend, weights),
               "sessions_by_count": lambda: {str(n): sessions_decode(backend, weights, count=n, steps=64)
                                             for n in (4, 8)}}
        print(json.dumps({args.extra_only: run[args.extra_only]()}), flush=True)
        backend.close()
        return 0
    prefix = np.random.default_rng(0).standard_normal((PREFIX, cfg.width)).astype(np.float32)

    backend = HipBackend(0)
    dec = HipDecoder(backend, weights, capacity=2048)
    persistent = dec.persistent
    # Warm-up pass: prefill, then `warmup` untimed decode steps.
    dec.decode(prefix, PREFIX)
    warm_tokens = dec.generate(args.warmup) if args.warmup else np.array([], dtype=np.int32)
    # Timed pass from the same state: reset, prefill (untimed), K timed steps.
    dec.reset()
    dec.decode(prefix, PREFIX)
    device.synchronize()
    start, end = device.Event(), device.Event()
    t0 = time.perf_counter()
    start.record(backend.stream)
    tokens = dec.generate(args.steps)
    end.record(backend.stream)
    end.synchronize()
    wall = time.perf_counter() - t0
    device.synchronize()
    gpu_ms = start.elapsed_ms(end)
    seconds = max(gpu_ms / 1000.0, 1e-9)
    tok_s = args.steps / seconds
    deterministic = bool(np.array_equal(tokens[: len(warm_tokens)], warm_tokens))

    weight_bytes = cfg.weight_bytes_per_token()
    kv_bytes = sum(114688 * (PREFIX + i + 1) for i in range(args.steps)) / max(args.steps, 1)
    step_bytes = weight_bytes + kv_bytes + 4 * (cfg.width * (2 * cfg.layers + 1) + 2 * cfg.head_size * cfg.layers)
    step_gbs = step_bytes * tok_s / 1e9

    gemv = gemv_roofline(backend, weights)
    dec.close()
    extra = {}
    if not args.no_extra:
        extra["gemv_sweep"] = gemv_sweep(backend)
        extra["float_gemv_sweep"] = float_gemv_sweep(backend)
        extra["encoder_float"] = encoder_float(backend)
        extra["prefill"] = prefill_ttft(backend, weights)
        extra["long_kv"] = long_kv(backend, weights)
        extra["sessions"] = sessions_decode(backend, weights,
                                            check=None if args.no_cpu else min(16, os.cpu_count() or 1))
        oracle_tokens = extra["sessions"].get("oracle_check", {}).pop("_tokens", None)
        extra["sessions"]["by_count"] = {str(n): sessions_decode(backend, weights, count=n, steps=64)
                                         for n in (4, 8)}
        extra["step_batcher"] = step_batcher_decode(backend, weights, expected=oracle_tokens)
        if not args.no_cpu:
            extra["cpu_baselines"] = cpu_extra_baselines(weights, min(16, os.cpu_count() or 1))
    backend.close()

    baseline = None
    if not args.no_cpu:
        # The reference's default of 4 threads (FunAsr.cs:94), then every core
        # this process may use (at most the physical cores, and at most 16:
        # a single-GPU host's share of its cores).
        cpu = host_cpu()
        every = min(cpu["available_cpus"], cpu["physical_cores"] or cpu["available_cpus"], 16)
        runs = {}
        for label, threads in (("reference_default", 4), ("all_cores", every)):
            cpu_tok_s, used, cpu_seconds, passes = cpu_baseline(weights, prefix, args.cpu_tokens, threads,
                                                                args.cpu_seconds)
            runs[label] = {"value": round(cpu_tok_s, 3), "cores": used, "seconds": round(cpu_seconds, 1),
                           "passes": passes}
        main_run = runs["reference_default"]
        baseline = {"value": main_run["value"], "unit": "tok/s", "cores": main_run["cores"], "kind": "port",
                    "sample": f"oracle (C restatement of the reference x64 Q8_0 path), same weights and prefix: "
                              f"passes of {args.cpu_tokens} greedy decode steps from the post-prefill state "
                              f"(positions 150-{150 + args.cpu_tokens - 1}), about {args.cpu_seconds:.0f} s per "
                              f"thread count; value at the reference's default of 4 threads",
                    "all_cores": runs["all_cores"], "cpu": cpu}

    step_us = gpu_ms * 1000.0 / args.steps
    # HBM bytes per launch from the rocprofv3 FETCH_SIZE/WRITE_SIZE passes of
    # this kernel on this workload, scaled by the lm_head GEMV calibration.
    traffic = None
    try:
        with open(os.path.join(ROOT, "profiles", "decode_step_traffic.json")) as fh:
            recorded = json.load(fh)
        if persistent and recorded.get("kernel") == "decode_step_kernel":
            traffic = int(recorded["hbm_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        traffic = None
    if persistent:
        kernel = "decode_step_kernel (persistent: one launch per decoded token)"
    else:
        kernel = "decode step graph (multi-kernel path, one hipGraph per token)"

    line = {
        "metric": "decode tok/s Qwen3-0.6B Q8_0 bs=1; Q8_0 GEMV achieved HBM GB/s vs peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gpu_ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 dot / fp32 accumulate (Q8_0)",
        "data": "synthetic random-init weights (seed 0) and N(0,1) prefix",
        "config": {"workload": "qwen3-0.6b q8_0 greedy decode, batch 1, 150-row prefix, F16 KV",
                   "global_batch": 1, "prefix": PREFIX, "decode_steps": args.steps, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(step_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": ("recorded, not measured in this run: profiles/decode_step_traffic.json, "
                                        "rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes of decode_step_kernel on "
                                        "this workload, scaled by the same counters on the lm_head GEMV")
                                       if traffic is not None else None,
                     "kernel": kernel, "avg_us": round(step_us, 3),
                     "algorithmic_bytes_per_launch": int(step_bytes)},
        "gemv_lm_head": {"kernel": gemv["kernel"], "avg_us": round(gemv["avg_us"], 3),
                         "algorithmic_bytes": gemv["algorithmic_bytes"], "achieved_gbs": round(gemv["achieved_gbs"], 1),
                         "frac": round(gemv["achieved_gbs"] / HBM_PEAK_GBS, 4)},
        "decode_step": {"wall_s": round(wall, 4), "deterministic_vs_warmup": deterministic},
        "cpu_baseline": baseline,
    }
    line.update(extra)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())

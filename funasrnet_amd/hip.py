"""ctypes binding of the C ABI (include/funasr_hip.h) and a Python mirror of
the reference's backend seam.

``HipBackend`` has the reference's method names and contracts
(src/FunAsrNet/IQuantizedComputeBackend.cs:4-14,
IGroupedComputeBackend.cs:4-13): ``try_quantized_linear`` returns False and
leaves the output untouched when the library declines, raises ValueError on
shape mismatch (ArgumentException) and RuntimeError on device failure.
``HipDecoder`` mirrors QwenDecoder's public surface (Decode, Embed, Greedy,
Reset, RestorePrefix) over the device-resident decoder.

The library must be built (``funasrnet_amd.build.build()``); there is no CPU
fallback: a missing library or device is an error.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from .model import DecoderWeights, Q8Tensor

# The in-tree build; FUNASRNET_HIP_LIBRARY names another copy (absolute path),
# as the C# loader's resolver does.
LIBRARY = os.environ.get("FUNASRNET_HIP_LIBRARY") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                                   "libfunasr_hip.so")

OK, DECLINED = 0, 1
ERROR_ARGUMENT, ERROR_DEVICE, ERROR_DISPOSED, ERROR_STATE = -1, -2, -3, -4

_vp = ctypes.c_void_p
_f32p = ctypes.POINTER(ctypes.c_float)
_i8p = ctypes.POINTER(ctypes.c_int8)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u16p = ctypes.POINTER(ctypes.c_uint16)


class Q8Host(ctypes.Structure):
    _fields_ = [("quantized", _i8p), ("scales", _f32p), ("rows", ctypes.c_int), ("cols", ctypes.c_int),
                ("blocks", ctypes.POINTER(ctypes.c_uint8))]


class LayerHost(ctypes.Structure):
    _fields_ = [(n, Q8Host) for n in ("wq", "wk", "wv", "wo", "gate", "up", "down")] + [
        ("attn_norm", _f32p), ("q_norm", _f32p), ("k_norm", _f32p), ("ffn_norm", _f32p)]


class DecoderConfigC(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("width", "heads", "kv_heads", "head_size", "layers", "ffn", "vocab")] + [
        ("eps", ctypes.c_float), ("rope_base", ctypes.c_float), ("capacity", ctypes.c_int)]


class CallStats(ctypes.Structure):
    """fah_call_stats: one seam entry point's counters."""
    _fields_ = [(n, ctypes.c_int64) for n in ("calls", "declined", "operations", "uploaded_bytes",
                                               "downloaded_bytes")] + [
        ("device_ms", ctypes.c_double), ("total_ms", ctypes.c_double)]


# Seam entry points in fah_context_statistics order (FAH_CALL_*).
CALL_KINDS = ("quantized_linear", "quantized_linear_noalloc", "linear_many", "linear", "relu_projection", "attention")
CALL_OBSERVER = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_double, ctypes.c_double)

# Every symbol of include/funasr_hip.h with its signature.
SIGNATURES = {
    "fah_context_statistics": (ctypes.c_int, [_vp, ctypes.POINTER(CallStats), ctypes.c_int]),
    "fah_context_reset_statistics": (ctypes.c_int, [_vp]),
    "fah_context_set_call_observer": (ctypes.c_int, [_vp, CALL_OBSERVER, _vp]),
    "fah_abi_version": (ctypes.c_int, []),
    "fah_last_error": (ctypes.c_char_p, []),
    "fah_device_count": (ctypes.c_int, []),
    "fah_context_create": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(_vp)]),
    "fah_context_destroy": (ctypes.c_int, [_vp]),
    "fah_context_synchronize": (ctypes.c_int, [_vp]),
    "fah_context_name": (ctypes.c_char_p, [_vp]),
    "fah_context_set_minimum_operations": (ctypes.c_int, [_vp, ctypes.c_int64]),
    "fah_context_stream": (_vp, [_vp]),
    "fah_weight_q8_upload": (ctypes.c_int, [_vp, _i8p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.POINTER(_vp)]),
    "fah_weight_q8_upload_blocks": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_uint8), ctypes.c_int, ctypes.c_int,
                                                   ctypes.POINTER(_vp)]),
    "fah_weight_f32_upload": (ctypes.c_int, [_vp, _f32p, ctypes.c_int, ctypes.c_int, ctypes.POINTER(_vp)]),
    "fah_weight_release": (ctypes.c_int, [_vp]),
    "fah_linear": (ctypes.c_int, [_vp, _f32p, ctypes.c_int, _vp, _f32p, _f32p]),
    "fah_relu_projection": (ctypes.c_int, [_vp, _f32p, ctypes.c_int, _vp, _f32p, _vp, _f32p, _f32p]),
    "fah_attention": (ctypes.c_int, [_vp, _f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p]),
    "fah_weight_device_bytes": (ctypes.c_int64, [_vp]),
    "fah_quantized_linear": (ctypes.c_int, [_vp, _f32p, ctypes.c_int, _vp, _f32p, _f32p]),
    "fah_quantized_linear_noalloc": (ctypes.c_int, [_vp, _f32p, ctypes.c_int, _vp, _f32p, _f32p]),
    "fah_linear_many": (ctypes.c_int, [_vp, _f32p, ctypes.c_int, ctypes.POINTER(_vp), ctypes.c_int,
                                       ctypes.POINTER(_f32p)]),
    "fah_quantize_device": (ctypes.c_int, [_vp, _vp, ctypes.c_int64, _vp, _vp]),
    "fah_rms_norm_device": (ctypes.c_int, [_vp, _vp, ctypes.c_int, ctypes.c_int, _vp, ctypes.c_float, _vp]),
    "fah_q8_gemv_device": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_int, _vp, _vp]),
    "fah_q8_block_dots_device": (ctypes.c_int, [_vp, _vp, _vp, _vp]),
    "fah_linear_device": (ctypes.c_int, [_vp, _vp, ctypes.c_int, _vp, _vp, _vp]),
    "fah_attention_device": (ctypes.c_int, [_vp, _vp, _vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp]),
    "fah_decoder_create": (ctypes.c_int, [_vp, ctypes.POINTER(DecoderConfigC), ctypes.POINTER(LayerHost),
                                          ctypes.POINTER(Q8Host), ctypes.POINTER(Q8Host), _f32p,
                                          ctypes.POINTER(_vp)]),
    "fah_decoder_destroy": (ctypes.c_int, [_vp]),
    "fah_decoder_set_position": (ctypes.c_int, [_vp, ctypes.c_int]),
    "fah_decoder_position": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_int)]),
    "fah_decoder_decode": (ctypes.c_int, [_vp, _f32p, ctypes.c_int, _f32p]),
    "fah_decoder_embed": (ctypes.c_int, [_vp, _i32p, ctypes.c_int, _f32p]),
    "fah_decoder_greedy": (ctypes.c_int, [_vp, _i32p]),
    "fah_decoder_generate": (ctypes.c_int, [_vp, ctypes.c_int, _i32p]),
    "fah_decoder_create_session": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.POINTER(_vp)]),
    "fah_decoder_generate_sessions": (ctypes.c_int, [ctypes.POINTER(_vp), ctypes.c_int, ctypes.c_int, _i32p]),
    "fah_batcher_create": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, ctypes.POINTER(_vp)]),
    "fah_batcher_destroy": (ctypes.c_int, [_vp]),
    "fah_batcher_join": (ctypes.c_int, [_vp, _vp]),
    "fah_batcher_leave": (ctypes.c_int, [_vp, _vp]),
    "fah_batcher_step": (ctypes.c_int, [_vp, _vp, _i32p]),
    "fah_batcher_stats": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)]),
    "fah_decoder_kv_write": (ctypes.c_int, [_vp, ctypes.c_int, _u16p, _u16p, ctypes.c_int]),
    "fah_decoder_kv_read": (ctypes.c_int, [_vp, ctypes.c_int, _u16p, _u16p, ctypes.c_int]),
    "fah_decoder_weight_bytes": (ctypes.c_int64, [_vp]),
    "fah_decoder_persistent": (ctypes.c_int, [_vp]),
    "fah_decoder_trace": (ctypes.c_int, [_vp, ctypes.c_int, _f32p, ctypes.c_int]),
    "fah_decoder_timeline": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_uint64), ctypes.c_int]),
    "fah_decoder_fail_next_step": (ctypes.c_int, [_vp]),
    "fah_decoder_attention_time": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int)]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load the in-tree HIP library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            raise RuntimeError(f"{LIBRARY} is missing: build it with funasrnet_amd.build.build()")
        lib = ctypes.CDLL(LIBRARY)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def _p(a: np.ndarray, ctype):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def _raise(rc: int):
    msg = load().fah_last_error().decode()
    if rc == ERROR_ARGUMENT:
        raise ValueError(msg)
    if rc == ERROR_DISPOSED:
        raise RuntimeError("disposed: " + msg)
    raise RuntimeError(msg)


def _check(rc: int) -> int:
    if rc < 0:
        _raise(rc)
    return rc


def device_count() -> int:
    return load().fah_device_count()


class HipWeight:
    """Device copy of a Q8_0 matrix (Weight.Quantized / Weight.Scales)."""

    def __init__(self, backend: "HipBackend", tensor: Q8Tensor):
        self.rows, self.columns = tensor.rows, tensor.columns
        self._backend = backend
        h = _vp()
        if tensor.quantized is None:
            raw = np.ascontiguousarray(tensor.blocks, dtype=np.uint8)
            _check(load().fah_weight_q8_upload_blocks(backend.handle, _p(raw, ctypes.c_uint8), self.rows,
                                                      self.columns, ctypes.byref(h)))
        else:
            q = np.ascontiguousarray(tensor.quantized, dtype=np.int8)
            s = np.ascontiguousarray(tensor.scales, dtype=np.float32)
            _check(load().fah_weight_q8_upload(backend.handle, _p(q, ctypes.c_int8), _p(s, ctypes.c_float), self.rows,
                                               self.columns, ctypes.byref(h)))
        self.handle = h

    @property
    def device_bytes(self) -> int:
        return load().fah_weight_device_bytes(self.handle)

    def close(self):
        if self.handle:
            load().fah_weight_release(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipFloatWeight:
    """Device copy of an FP32 matrix (Weight.Values, rows x columns)."""

    def __init__(self, backend: "HipBackend", values: np.ndarray):
        v = np.ascontiguousarray(values, dtype=np.float32)
        if v.ndim != 2:
            raise ValueError("FP32 weight must be a rows x columns matrix")
        self.rows, self.columns = v.shape
        h = _vp()
        _check(load().fah_weight_f32_upload(backend.handle, _p(v, ctypes.c_float), self.rows, self.columns,
                                            ctypes.byref(h)))
        self.handle = h

    @property
    def device_bytes(self) -> int:
        return load().fah_weight_device_bytes(self.handle)

    def close(self):
        if self.handle:
            load().fah_weight_release(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipBackend:
    """IFloatComputeBackend (TryLinear), IQuantizedComputeBackend,
    IGroupedComputeBackend, IReluProjectionBackend and
    IAttentionComputeBackend over one context."""

    def __init__(self, device: int = 0, minimum_operations: int | None = None):
        h = _vp()
        _check(load().fah_context_create(device, ctypes.byref(h)))
        self.handle = h
        self._weights = {}
        if minimum_operations is not None:
            _check(load().fah_context_set_minimum_operations(h, minimum_operations))

    @property
    def name(self) -> str:
        return load().fah_context_name(self.handle).decode()

    @property
    def stream(self) -> int:
        return load().fah_context_stream(self.handle) or 0

    def synchronize(self):
        _check(load().fah_context_synchronize(self.handle))

    def statistics(self) -> dict:
        """Per seam entry point: calls, declined, operations, uploaded and
        downloaded bytes, device and wall milliseconds
        (VulkanFloatBackend.Statistics() analogue)."""
        recs = (CallStats * len(CALL_KINDS))()
        _check(load().fah_context_statistics(self.handle, recs, len(CALL_KINDS)))
        return {k: {f: getattr(r, f) for f, _ in CallStats._fields_} for k, r in zip(CALL_KINDS, recs)}

    def reset_statistics(self):
        _check(load().fah_context_reset_statistics(self.handle))

    def set_call_observer(self, fn):
        """fn(kind_name, frames, cols, rows, device_ms, total_ms) after every
        seam call that ran on the device (TensorMath.LinearMeasured analogue);
        None removes it."""
        if fn is None:
            self._observer = None
            _check(load().fah_context_set_call_observer(self.handle, CALL_OBSERVER(), None))
            return

        def trampoline(_user, kind, frames, cols, rows, device_ms, total_ms):
            fn(CALL_KINDS[kind], frames, cols, rows, device_ms, total_ms)

        self._observer = CALL_OBSERVER(trampoline)  # kept alive while installed
        _check(load().fah_context_set_call_observer(self.handle, self._observer, None))

    def weight(self, tensor: Q8Tensor) -> HipWeight:
        """Device weight cached by tensor identity (the reference keys its
        cache on the managed array, VulkanFloatBackend.cs:242-283)."""
        key = id(tensor)
        if key not in self._weights:
            self._weights[key] = (tensor, HipWeight(self, tensor))
        return self._weights[key][1]

    def float_weight(self, values: np.ndarray) -> HipFloatWeight:
        """Device FP32 weight cached by array identity (VulkanFloatBackend.cs:242-283)."""
        key = ("f32", id(values))
        if key not in self._weights:
            self._weights[key] = (values, HipFloatWeight(self, values))
        return self._weights[key][1]

    def try_linear(self, input: np.ndarray, frames: int, weight: np.ndarray, bias, output: np.ndarray) -> bool:
        """IFloatComputeBackend.TryLinear: output[frames, rows] = input W^T + bias
        for an FP32 weight [rows, columns]; False (output untouched) when declined."""
        w = self.float_weight(weight)
        x = np.ascontiguousarray(input, dtype=np.float32)
        if x.size != frames * w.columns or output.size != frames * w.rows:
            raise ValueError("GPU linear projection shape mismatch")
        out = np.empty(frames * w.rows, dtype=np.float32)
        b = None if bias is None else _p(np.ascontiguousarray(bias, dtype=np.float32), ctypes.c_float)
        rc = _check(load().fah_linear(self.handle, _p(x, ctypes.c_float), frames, w.handle, b, _p(out, ctypes.c_float)))
        if rc == DECLINED:
            return False
        output.reshape(-1)[:] = out
        return True

    def try_relu_projection(self, input: np.ndarray, frames: int, first: np.ndarray, first_bias, second: np.ndarray,
                            second_bias, output: np.ndarray) -> bool:
        """IReluProjectionBackend.TryReluProjection: ReLU(x W1^T + b1) W2^T + b2."""
        w1, w2 = self.float_weight(first), self.float_weight(second)
        x = np.ascontiguousarray(input, dtype=np.float32)
        if x.size != frames * w1.columns or output.size != frames * w2.rows:
            raise ValueError("ReLU projection input, weight or output shape mismatch")
        out = np.empty(frames * w2.rows, dtype=np.float32)
        b1 = None if first_bias is None else _p(np.ascontiguousarray(first_bias, dtype=np.float32), ctypes.c_float)
        b2 = None if second_bias is None else _p(np.ascontiguousarray(second_bias, dtype=np.float32), ctypes.c_float)
        rc = _check(load().fah_relu_projection(self.handle, _p(x, ctypes.c_float), frames, w1.handle, b1, w2.handle, b2,
                                               _p(out, ctypes.c_float)))
        if rc == DECLINED:
            return False
        output.reshape(-1)[:] = out
        return True

    def try_attention(self, query: np.ndarray, key: np.ndarray, value: np.ndarray, frames: int, width: int,
                      heads: int, output: np.ndarray) -> bool:
        """IAttentionComputeBackend.TryAttention over [frames, width] rows."""
        q = np.ascontiguousarray(query, dtype=np.float32)
        k = np.ascontiguousarray(key, dtype=np.float32)
        v = np.ascontiguousarray(value, dtype=np.float32)
        count = frames * width
        if min(frames, width, heads) < 1 or width % heads or width // heads > 256 or frames > 4096:
            return False
        if q.size != count or k.size != count or v.size != count or output.size != count:
            raise ValueError("GPU attention input/output shapes differ")
        out = np.empty(count, dtype=np.float32)
        rc = _check(load().fah_attention(self.handle, _p(q, ctypes.c_float), _p(k, ctypes.c_float),
                                         _p(v, ctypes.c_float), frames, width, heads, _p(out, ctypes.c_float)))
        if rc == DECLINED:
            return False
        output.reshape(-1)[:] = out
        return True

    def try_quantized_linear(self, input: np.ndarray, frames: int, weight: Q8Tensor, bias, output: np.ndarray) -> bool:
        w = self.weight(weight)
        x = np.ascontiguousarray(input, dtype=np.float32)
        if x.size != frames * w.columns or output.size != frames * w.rows:
            raise ValueError("Q8 GPU projection shape mismatch")
        out = np.empty(frames * w.rows, dtype=np.float32)
        b = None if bias is None else _p(np.ascontiguousarray(bias, dtype=np.float32), ctypes.c_float)
        rc = _check(load().fah_quantized_linear(self.handle, _p(x, ctypes.c_float), frames, w.handle, b,
                                                _p(out, ctypes.c_float)))
        if rc == DECLINED:
            return False
        output.reshape(-1)[:] = out
        return True

    def try_linear_many(self, input: np.ndarray, frames: int, weights: list):
        """IGroupedComputeBackend.TryLinearMany over Q8_0 tensors or FP32 arrays."""
        ws = [self.float_weight(t) if isinstance(t, np.ndarray) else self.weight(t) for t in weights]
        x = np.ascontiguousarray(input, dtype=np.float32)
        outs = [np.empty(frames * w.rows, dtype=np.float32) for w in ws]
        handles = (_vp * len(ws))(*[w.handle for w in ws])
        ptrs = (_f32p * len(ws))(*[_p(o, ctypes.c_float) for o in outs])
        rc = _check(load().fah_linear_many(self.handle, _p(x, ctypes.c_float), frames, handles, len(ws), ptrs))
        return None if rc == DECLINED else outs

    # device-pointer entry points (pointers are integers, e.g. torch data_ptr())
    def quantize_device(self, x_ptr: int, n: int, q_ptr: int, s_ptr: int):
        _check(load().fah_quantize_device(self.handle, x_ptr, n, q_ptr, s_ptr))

    def rms_norm_device(self, x_ptr: int, rows: int, width: int, scale_ptr: int, eps: float, y_ptr: int):
        """RMSNorm rows on the device (QwenDecoder.Norm's arithmetic)."""
        _check(load().fah_rms_norm_device(self.handle, x_ptr, rows, width, scale_ptr, eps, y_ptr))

    def gemv_device(self, q_ptr: int, s_ptr: int, frames: int, weight: HipWeight, out_ptr: int) -> int:
        return _check(load().fah_q8_gemv_device(self.handle, q_ptr, s_ptr, frames, weight.handle, out_ptr))

    def linear_device(self, x_ptr: int, frames: int, weight: HipFloatWeight, bias_ptr, out_ptr: int) -> int:
        return _check(load().fah_linear_device(self.handle, x_ptr, frames, weight.handle, bias_ptr, out_ptr))

    def attention_device(self, q_ptr: int, k_ptr: int, v_ptr: int, frames: int, width: int, heads: int,
                         out_ptr: int) -> int:
        return _check(load().fah_attention_device(self.handle, q_ptr, k_ptr, v_ptr, frames, width, heads, out_ptr))

    def block_dots_device(self, q_ptr: int, weight: HipWeight, dots_ptr: int):
        _check(load().fah_q8_block_dots_device(self.handle, q_ptr, weight.handle, dots_ptr))

    def close(self):
        for _, w in self._weights.values():
            w.close()
        self._weights.clear()
        if self.handle:
            load().fah_context_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipDecoder:
    """QwenDecoder (src/FunAsrNet/QwenDecoder.cs) on the device."""

    def __init__(self, backend: HipBackend, weights: DecoderWeights | None, capacity: int = 2048,
                 parent: "HipDecoder | None" = None):
        if parent is not None:
            # A session over the parent's device weights (fah_decoder_create_session).
            h = _vp()
            _check(load().fah_decoder_create_session(parent.handle, capacity, ctypes.byref(h)))
            self.handle = h
            self.config = parent.config
            self.capacity = capacity
            self.backend = backend
            self.parent = parent
            return
        c = weights.config
        keep = []

        def q8(t: Q8Tensor) -> Q8Host:
            if t.quantized is None:  # GGUF blocks, split on the device
                raw = np.ascontiguousarray(t.blocks, dtype=np.uint8)
                keep.append(raw)
                return Q8Host(None, None, t.rows, t.columns, _p(raw, ctypes.c_uint8))
            q = np.ascontiguousarray(t.quantized, dtype=np.int8)
            s = np.ascontiguousarray(t.scales, dtype=np.float32)
            keep.extend([q, s])
            return Q8Host(_p(q, ctypes.c_int8), _p(s, ctypes.c_float), t.rows, t.columns, None)

        def f32(a):
            a = np.ascontiguousarray(a, dtype=np.float32)
            keep.append(a)
            return _p(a, ctypes.c_float)

        layers = (LayerHost * c.layers)()
        for i, L in enumerate(weights.layers):
            layers[i] = LayerHost(q8(L.wq), q8(L.wk), q8(L.wv), q8(L.wo), q8(L.gate), q8(L.up), q8(L.down),
                                  f32(L.attn_norm), f32(L.q_norm), f32(L.k_norm), f32(L.ffn_norm))
        cfg = DecoderConfigC(c.width, c.heads, c.kv_heads, c.head_size, c.layers, c.ffn, c.vocab, c.eps, c.rope_base,
                             capacity)
        embd = q8(weights.token_embd)
        output = q8(weights.output) if weights.output is not None else None
        h = _vp()
        _check(load().fah_decoder_create(backend.handle, ctypes.byref(cfg), layers, ctypes.byref(embd),
                                         ctypes.byref(output) if output is not None else None,
                                         f32(weights.output_norm), ctypes.byref(h)))
        self.handle = h
        self.config = c
        self.capacity = capacity
        self.backend = backend
        self.parent = None

    def session(self, capacity: int | None = None) -> "HipDecoder":
        """A new session sharing this decoder's device weights, with its own
        KV cache of `capacity` positions (default: this decoder's)."""
        return HipDecoder(self.backend, None, capacity or self.capacity, parent=self)

    def close(self):
        if self.handle:
            load().fah_decoder_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def position(self) -> int:
        v = ctypes.c_int()
        _check(load().fah_decoder_position(self.handle, ctypes.byref(v)))
        return v.value

    def reset(self):
        """QwenDecoder.Reset (QwenDecoder.cs:117)."""
        self.set_position(0)

    def set_position(self, position: int):
        """QwenDecoder.RestorePrefix (QwenDecoder.cs:137) for any cached length."""
        _check(load().fah_decoder_set_position(self.handle, position))

    def decode(self, embeddings: np.ndarray, frames: int, output_logits: bool = True):
        x = np.ascontiguousarray(embeddings, dtype=np.float32)
        if x.size != frames * self.config.width:
            raise ValueError("Decoder context exhausted or invalid embeddings")
        logits = np.empty(self.config.vocab, dtype=np.float32) if output_logits else None
        _check(load().fah_decoder_decode(self.handle, _p(x, ctypes.c_float), frames,
                                         None if logits is None else _p(logits, ctypes.c_float)))
        return logits

    def embed(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty((t.size, self.config.width), dtype=np.float32)
        _check(load().fah_decoder_embed(self.handle, _p(t, ctypes.c_int32), t.size, _p(out, ctypes.c_float)))
        return out

    def greedy(self) -> int:
        v = ctypes.c_int32()
        _check(load().fah_decoder_greedy(self.handle, ctypes.byref(v)))
        return v.value

    def generate(self, steps: int) -> np.ndarray:
        tokens = np.empty(max(steps, 1), dtype=np.int32)
        _check(load().fah_decoder_generate(self.handle, steps, _p(tokens, ctypes.c_int32)))
        return tokens[:steps]

    @staticmethod
    def generate_sessions(sessions, steps: int) -> np.ndarray:
        """Lock-step greedy decode of sessions that share one weight set:
        tokens [len(sessions), steps], row i for sessions[i]."""
        count = len(sessions)
        handles = (_vp * count)(*[d.handle for d in sessions])
        tokens = np.empty((count, max(steps, 1)), dtype=np.int32)
        _check(load().fah_decoder_generate_sessions(handles, count, steps, _p(tokens, ctypes.c_int32)))
        return tokens[:, :steps]

    def kv_write(self, layer: int, keys_f16: np.ndarray, values_f16: np.ndarray):
        k = np.ascontiguousarray(keys_f16, dtype=np.float16).view(np.uint16)
        v = np.ascontiguousarray(values_f16, dtype=np.float16).view(np.uint16)
        width = self.config.kv_width
        positions = k.size // width
        _check(load().fah_decoder_kv_write(self.handle, layer, _p(k, ctypes.c_uint16), _p(v, ctypes.c_uint16),
                                           positions))

    def kv_read(self, layer: int, positions: int):
        width = self.config.kv_width
        k = np.empty(positions * width, dtype=np.uint16)
        v = np.empty(positions * width, dtype=np.uint16)
        _check(load().fah_decoder_kv_read(self.handle, layer, _p(k, ctypes.c_uint16), _p(v, ctypes.c_uint16),
                                          positions))
        return k.view(np.float16), v.view(np.float16)

    @property
    def weight_bytes(self) -> int:
        return load().fah_decoder_weight_bytes(self.handle)

    TRACE = {"x": 0, "qkv": 1, "attn": 2, "a": 3, "h": 4}

    def trace(self, name: str) -> np.ndarray:
        """Last-layer activation snapshot (QwenDecoder.Trace analogue)."""
        c = self.config
        size = {"x": c.width, "qkv": c.q_width + 2 * c.kv_width, "attn": c.q_width, "a": c.width, "h": c.ffn}[name]
        out = np.empty(size, dtype=np.float32)
        _check(load().fah_decoder_trace(self.handle, self.TRACE[name], _p(out, ctypes.c_float), size))
        return out

    def timeline(self):
        """[workgroups, 480] device-clock stamps of the last persistent step, or None."""
        out = np.zeros(256 * 480, dtype=np.uint64)
        rc = _check(load().fah_decoder_timeline(self.handle, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)), out.size))
        return None if rc == DECLINED else out.reshape(256, 480)

    def attention_time(self):
        """(milliseconds, steps) of attention kernels since the last call, or
        None unless the decoder was created with FAH_ATTENTION_TIMES=1."""
        ms, steps = ctypes.c_double(), ctypes.c_int()
        rc = _check(load().fah_decoder_attention_time(self.handle, ctypes.byref(ms), ctypes.byref(steps)))
        return None if rc == DECLINED else (ms.value, steps.value)

    @property
    def persistent(self) -> bool:
        return bool(load().fah_decoder_persistent(self.handle))


class HipStepBatcher:
    """Cross-context step batching over the sessions of one decoder
    (fah_batcher_*): worker threads each call step() for their own session
    once per token; concurrent steps run as one lock-step batch."""

    def __init__(self, parent: HipDecoder, max_positions: int, window_us: int = 200):
        h = _vp()
        _check(load().fah_batcher_create(parent.handle, max_positions, window_us, ctypes.byref(h)))
        self.handle = h
        self.parent = parent

    def join(self, session: HipDecoder):
        _check(load().fah_batcher_join(self.handle, session.handle))

    def leave(self, session: HipDecoder):
        _check(load().fah_batcher_leave(self.handle, session.handle))

    def step(self, session: HipDecoder) -> int:
        """One greedy step of `session` (its next token), batched with the
        steps other threads request meanwhile."""
        t = ctypes.c_int32()
        _check(load().fah_batcher_step(self.handle, session.handle, ctypes.byref(t)))
        return t.value

    def stats(self):
        """(batches run, session steps served)."""
        a, b = ctypes.c_int64(), ctypes.c_int64()
        _check(load().fah_batcher_stats(self.handle, ctypes.byref(a), ctypes.byref(b)))
        return a.value, b.value

    def close(self):
        if self.handle:
            _check(load().fah_batcher_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

"""ctypes wrapper over the CPU oracle (oracle/fah_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()``
and by bench.py's ``cpu_baseline`` leg, always as the reference the GPU
results are compared against or the timed CPU baseline, never as the product
path. The C source restates the reference's
x64 C# arithmetic; see the header of fah_oracle.h for which functions are
pinned by which independent checks.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(_HERE, "_build", "liboracle.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_i8p = ctypes.POINTER(ctypes.c_int8)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u8p = ctypes.POINTER(ctypes.c_uint8)


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc, no FMA contraction)."""
    args = ["make", "-C", _HERE]
    if force:
        args.append("-B")
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)
    return LIBRARY


class _Q8(ctypes.Structure):
    _fields_ = [("q", _i8p), ("scales", _f32p), ("rows", ctypes.c_int), ("cols", ctypes.c_int)]


class _Layer(ctypes.Structure):
    _fields_ = [(n, _Q8) for n in ("wq", "wk", "wv", "wo", "gate", "up", "down")] + [
        ("attn_norm", _f32p), ("q_norm", _f32p), ("k_norm", _f32p), ("ffn_norm", _f32p)]


class _Model(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("width", "heads", "kv_heads", "head_size", "layers", "ffn", "vocab")] + [
        ("eps", ctypes.c_float), ("rope_base", ctypes.c_float), ("layer", ctypes.POINTER(_Layer)),
        ("token_embd", _Q8), ("output", _Q8), ("output_norm", _f32p)]


def _load():
    if not os.path.exists(LIBRARY):
        build()
    lib = ctypes.CDLL(LIBRARY)
    sig = {
        "oracle_half_to_float": (ctypes.c_float, [ctypes.c_uint16]),
        "oracle_float_to_half": (ctypes.c_uint16, [ctypes.c_float]),
        "oracle_round_half": (ctypes.c_float, [ctypes.c_float]),
        "oracle_round_half_copy": (None, [_f32p, ctypes.c_int64, _f32p]),
        "oracle_exp": (ctypes.c_float, [ctypes.c_float]),
        "oracle_set_threads": (ctypes.c_int, [ctypes.c_int]),
        "oracle_unpack_q8": (ctypes.c_int, [_u8p, ctypes.c_int64, _i8p, _f32p]),
        "oracle_quantize": (ctypes.c_int, [_f32p, ctypes.c_int64, _i8p, _f32p]),
        "oracle_block_dot": (ctypes.c_int32, [_i8p, _i8p]),
        "oracle_q8_block_dots": (None, [_i8p, _i8p, ctypes.c_int, ctypes.c_int, _i32p]),
        "oracle_q8_gemv_quantized": (None, [_i8p, _f32p, ctypes.c_int, _i8p, _f32p, ctypes.c_int, ctypes.c_int, _f32p, _f32p]),
        "oracle_q8_linear": (ctypes.c_int, [_f32p, ctypes.c_int, _i8p, _f32p, ctypes.c_int, ctypes.c_int, _f32p, _f32p]),
        "oracle_embed_row": (None, [_i8p, _f32p, ctypes.c_int, ctypes.c_int, _f32p]),
        "oracle_rms_norm": (ctypes.c_int, [_f32p, ctypes.c_int64, ctypes.c_int, _f32p, ctypes.c_float, _f32p]),
        "oracle_rope_table": (None, [ctypes.c_int, ctypes.c_int, ctypes.c_float, _f32p, _f32p]),
        "oracle_rotate_half": (None, [_f32p, _f32p, _f32p, ctypes.c_int]),
        "oracle_softmax": (None, [_f32p, ctypes.c_int]),
        "oracle_silu_multiply": (None, [_f32p, _f32p, ctypes.c_int64]),
        "oracle_add": (None, [_f32p, _f32p, ctypes.c_int64]),
        "oracle_dot": (ctypes.c_float, [_f32p, _f32p, ctypes.c_int]),
        "oracle_greedy": (ctypes.c_int32, [_f32p, ctypes.c_int64]),
        "oracle_attention": (None, [_f32p, _f32p, _f32p] + [ctypes.c_int] * 5 + [_f32p]),
        "oracle_decoder_create": (ctypes.c_void_p, [ctypes.POINTER(_Model), ctypes.c_int]),
        "oracle_decoder_destroy": (None, [ctypes.c_void_p]),
        "oracle_decoder_reset": (None, [ctypes.c_void_p]),
        "oracle_decoder_position": (ctypes.c_int, [ctypes.c_void_p]),
        "oracle_decoder_set_position": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
        "oracle_decoder_decode": (ctypes.c_int, [ctypes.c_void_p, _f32p, ctypes.c_int, _f32p]),
        "oracle_decoder_embed": (ctypes.c_int, [ctypes.c_void_p, _i32p, ctypes.c_int, _f32p]),
        "oracle_decoder_keys": (_f32p, [ctypes.c_void_p, ctypes.c_int]),
        "oracle_decoder_values": (_f32p, [ctypes.c_void_p, ctypes.c_int]),
        "oracle_last_error": (ctypes.c_char_p, []),
        "oracle_decoder_capture_norms": (None, [ctypes.c_void_p, _f32p, ctypes.c_int64, _f32p, ctypes.c_int64]),
        "oracle_decoder_captured": (ctypes.c_int64, [ctypes.c_void_p, ctypes.c_int]),
        "oracle_sum_sq_gpu_tree": (ctypes.c_double, [_f32p, ctypes.c_int]),
        "oracle_sum_sq_reference": (ctypes.c_double, [_f32p, ctypes.c_int]),
        "oracle_rms_mean_settled": (ctypes.c_int, [ctypes.c_double, ctypes.c_int, _f32p]),
        "oracle_norm_order_stats": (ctypes.c_int, [_f32p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                                   ctypes.c_int64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_int64)]),
        "oracle_norm_order_find": (ctypes.c_int64, [_f32p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                                    ctypes.c_uint64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                                    _f32p]),
        "oracle_float_linear_f64": (None, [_f32p, ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_int, _f32p,
                                           ctypes.POINTER(ctypes.c_double)]),
        "oracle_attention_f64": (None, [_f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.POINTER(ctypes.c_double)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _p(a: np.ndarray, ctype):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def _check(rc: int):
    if rc != 0:
        raise ValueError(lib().oracle_last_error().decode())


def set_threads(threads: int) -> int:
    return lib().oracle_set_threads(int(threads))


def half_to_float(h: int) -> float:
    return lib().oracle_half_to_float(h)


def round_half(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().oracle_round_half_copy(_p(x, ctypes.c_float), x.size, _p(y, ctypes.c_float))
    return y


def exp(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    f = lib().oracle_exp
    return np.array([f(float(v)) for v in x.ravel()], dtype=np.float32).reshape(x.shape)


def unpack_q8(raw: np.ndarray, blocks: int):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    q = np.empty(blocks * 32, dtype=np.int8)
    s = np.empty(blocks, dtype=np.float32)
    _check(lib().oracle_unpack_q8(_p(raw, ctypes.c_uint8), blocks, _p(q, ctypes.c_int8), _p(s, ctypes.c_float)))
    return q, s


def quantize(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(x.shape, dtype=np.int8)
    s = np.empty(x.size // 32, dtype=np.float32)
    _check(lib().oracle_quantize(_p(x, ctypes.c_float), x.size, _p(q, ctypes.c_int8), _p(s, ctypes.c_float)))
    return q, s


def block_dots(xq: np.ndarray, wq: np.ndarray) -> np.ndarray:
    rows, cols = wq.shape
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    out = np.empty((rows, cols // 32), dtype=np.int32)
    lib().oracle_q8_block_dots(_p(xq, ctypes.c_int8), _p(wq, ctypes.c_int8), rows, cols, _p(out, ctypes.c_int32))
    return out


def gemv_quantized(xq, xs, wq, ws, bias=None) -> np.ndarray:
    rows, cols = wq.shape
    xq = np.ascontiguousarray(xq, dtype=np.int8).reshape(-1, cols)
    frames = xq.shape[0]
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    ws = np.ascontiguousarray(ws, dtype=np.float32)
    out = np.empty((frames, rows), dtype=np.float32)
    b = None if bias is None else _p(np.ascontiguousarray(bias, dtype=np.float32), ctypes.c_float)
    lib().oracle_q8_gemv_quantized(_p(xq, ctypes.c_int8), _p(xs, ctypes.c_float), frames, _p(wq, ctypes.c_int8),
                                   _p(ws, ctypes.c_float), rows, cols, b, _p(out, ctypes.c_float))
    return out


def linear(x, wq, ws, bias=None) -> np.ndarray:
    """TensorMath.Linear for Q8 weights: wq [rows, cols] int8, ws [rows, cols/32]."""
    rows, cols = wq.shape
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, cols)
    frames = x.shape[0]
    out = np.empty((frames, rows), dtype=np.float32)
    bias_arr = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    b = None if bias_arr is None else _p(bias_arr, ctypes.c_float)
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    ws = np.ascontiguousarray(ws, dtype=np.float32)
    _check(lib().oracle_q8_linear(_p(x, ctypes.c_float), frames, _p(wq, ctypes.c_int8), _p(ws, ctypes.c_float),
                                  rows, cols, b, _p(out, ctypes.c_float)))
    return out


def rms_norm(x, width: int, scale, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    scale = np.ascontiguousarray(scale, dtype=np.float32)
    y = np.empty_like(x)
    _check(lib().oracle_rms_norm(_p(x, ctypes.c_float), x.size, width, _p(scale, ctypes.c_float), eps, _p(y, ctypes.c_float)))
    return y


def rope_table(capacity: int, head_size: int, base: float):
    half = head_size // 2
    c = np.empty((capacity, half), dtype=np.float32)
    s = np.empty((capacity, half), dtype=np.float32)
    lib().oracle_rope_table(capacity, head_size, base, _p(c, ctypes.c_float), _p(s, ctypes.c_float))
    return c, s


def rotate_half(x, cosine, sine) -> np.ndarray:
    x = np.array(x, dtype=np.float32, copy=True)
    cosine = np.ascontiguousarray(cosine, dtype=np.float32)
    sine = np.ascontiguousarray(sine, dtype=np.float32)
    lib().oracle_rotate_half(_p(x, ctypes.c_float), _p(cosine, ctypes.c_float), _p(sine, ctypes.c_float), cosine.size)
    return x


def softmax(x) -> np.ndarray:
    x = np.array(x, dtype=np.float32, copy=True)
    lib().oracle_softmax(_p(x, ctypes.c_float), x.size)
    return x


def silu_multiply(gate, up) -> np.ndarray:
    g = np.array(gate, dtype=np.float32, copy=True)
    u = np.ascontiguousarray(up, dtype=np.float32)
    lib().oracle_silu_multiply(_p(g, ctypes.c_float), _p(u, ctypes.c_float), g.size)
    return g


def dot(a, b) -> float:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return lib().oracle_dot(_p(a, ctypes.c_float), _p(b, ctypes.c_float), a.size)


def float_linear_f64(x, frames: int, w, bias=None) -> np.ndarray:
    """y[frames, rows] = x W^T (+ bias) in double (FP32 projection reference)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    out = np.empty(frames * rows, dtype=np.float64)
    b = None if bias is None else _p(np.ascontiguousarray(bias, dtype=np.float32), ctypes.c_float)
    lib().oracle_float_linear_f64(_p(x, ctypes.c_float), frames, cols, _p(w, ctypes.c_float), rows, b,
                                  out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
    return out.reshape(frames, rows)


def attention_f64(q, k, v, frames: int, width: int, heads: int) -> np.ndarray:
    """Non-causal multi-head attention in double over [frames, width] rows."""
    q, k, v = (np.ascontiguousarray(a, dtype=np.float32).reshape(-1) for a in (q, k, v))
    out = np.empty(frames * width, dtype=np.float64)
    lib().oracle_attention_f64(_p(q, ctypes.c_float), _p(k, ctypes.c_float), _p(v, ctypes.c_float), frames, width,
                               heads, out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
    return out.reshape(frames, width)


def sum_sq_gpu_tree(x) -> float:
    """The GPU kernels' pairwise-tree square sum of one RMSNorm row."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    return lib().oracle_sum_sq_gpu_tree(_p(x, ctypes.c_float), x.size)


def sum_sq_reference(x) -> float:
    """The reference's four-chain square sum (TensorMath.Elementwise.cs:58-71)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    return lib().oracle_sum_sq_reference(_p(x, ctypes.c_float), x.size)


def rms_mean_settled(tree: float, width: int):
    """(settled, mean) of the GPU's exactness test on a tree sum."""
    m = np.zeros(1, np.float32)
    ok = lib().oracle_rms_mean_settled(float(tree), width, _p(m, ctypes.c_float))
    return bool(ok), m[0]


def norm_order_stats(pool, width: int, rows: int, seed: int, rowwise: bool = False):
    """Counts over `rows` sample rows drawn from `pool`: rows, rows whose
    tree float mean differs from the reference's, rows the GPU test leaves to
    the reference's order, rows it settles wrongly (must be 0). A flat pool
    (a power-of-two number of values) is mixed into rows; a rowwise pool
    [n, width] gives whole rows. Values get random low mantissa bits."""
    pool = np.ascontiguousarray(pool, dtype=np.float32)
    counts = (ctypes.c_int64 * 4)()
    _check(lib().oracle_norm_order_stats(_p(pool, ctypes.c_float), pool.size, width, int(rowwise), rows, seed,
                                         counts))
    return tuple(counts)


def norm_order_find(pool, width: int, seed: int, start: int, rows: int, want: int,
                    rowwise: bool = False) -> np.ndarray:
    """Sample rows (same draw as norm_order_stats) whose tree float mean
    differs from the reference's."""
    pool = np.ascontiguousarray(pool, dtype=np.float32)
    out = np.zeros((want, width), np.float32)
    n = lib().oracle_norm_order_find(_p(pool, ctypes.c_float), pool.size, width, int(rowwise), seed, start, rows,
                                     want, _p(out, ctypes.c_float))
    return out[:n]


def greedy(logits) -> int:
    x = np.ascontiguousarray(logits, dtype=np.float32)
    return lib().oracle_greedy(_p(x, ctypes.c_float), x.size)


def attention(q, kcache, vcache, frames, position, heads, kv_heads, head_size) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(kcache, dtype=np.float32)
    v = np.ascontiguousarray(vcache, dtype=np.float32)
    out = np.empty(frames * heads * head_size, dtype=np.float32)
    lib().oracle_attention(_p(q, ctypes.c_float), _p(k, ctypes.c_float), _p(v, ctypes.c_float),
                           frames, position, heads, kv_heads, head_size, _p(out, ctypes.c_float))
    return out


@dataclass
class _Keep:
    arrays: list


class Decoder:
    """QwenDecoder (src/FunAsrNet/QwenDecoder.cs:9-385) restated in C.

    ``weights`` is a :class:`funasrnet_amd.model.DecoderWeights`-like object
    exposing ``config`` and the per-tensor (q, scales) arrays.
    """

    def __init__(self, weights, capacity: int = 2048):
        cfg = weights.config
        keep = []

        def q8(w):
            q = np.ascontiguousarray(w.quantized, dtype=np.int8)
            s = np.ascontiguousarray(w.scales, dtype=np.float32)
            keep.extend([q, s])
            return _Q8(_p(q, ctypes.c_int8), _p(s, ctypes.c_float), w.rows, w.columns)

        def f32(a):
            a = np.ascontiguousarray(a, dtype=np.float32)
            keep.append(a)
            return _p(a, ctypes.c_float)

        layers = (_Layer * cfg.layers)()
        for i in range(cfg.layers):
            L = weights.layers[i]
            layers[i] = _Layer(q8(L.wq), q8(L.wk), q8(L.wv), q8(L.wo), q8(L.gate), q8(L.up), q8(L.down),
                               f32(L.attn_norm), f32(L.q_norm), f32(L.k_norm), f32(L.ffn_norm))
        output = q8(weights.output) if weights.output is not None else _Q8(None, None, 0, 0)
        self._model = _Model(cfg.width, cfg.heads, cfg.kv_heads, cfg.head_size, cfg.layers, cfg.ffn, cfg.vocab,
                             cfg.eps, cfg.rope_base, layers, q8(weights.token_embd), output, f32(weights.output_norm))
        self._keep = _Keep(keep + [layers])
        self.config = cfg
        self.capacity = capacity
        self._handle = lib().oracle_decoder_create(ctypes.byref(self._model), capacity)
        if not self._handle:
            raise ValueError(lib().oracle_last_error().decode())

    def close(self):
        if self._handle:
            lib().oracle_decoder_destroy(self._handle)
            self._handle = None

    def __del__(self):
        self.close()

    def reset(self):
        lib().oracle_decoder_reset(self._handle)

    @property
    def position(self) -> int:
        return lib().oracle_decoder_position(self._handle)

    def set_position(self, position: int):
        _check(lib().oracle_decoder_set_position(self._handle, position))

    def embed(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty((t.size, self.config.width), dtype=np.float32)
        _check(lib().oracle_decoder_embed(self._handle, _p(t, ctypes.c_int32), t.size, _p(out, ctypes.c_float)))
        return out

    def decode(self, embeddings, frames: int, output_logits: bool = True):
        x = np.ascontiguousarray(embeddings, dtype=np.float32)
        logits = np.empty(self.config.vocab, dtype=np.float32) if output_logits else None
        _check(lib().oracle_decoder_decode(self._handle, _p(x, ctypes.c_float), frames,
                                           None if logits is None else _p(logits, ctypes.c_float)))
        return logits

    def capture_norms(self, wide_rows: int, head_rows: int):
        """Record the input rows of the next decodes' RMSNorms (width-wide
        and per-head), up to the given counts; returns the two arrays, filled
        as the decodes run (see captured())."""
        cfg = self.config
        self._cap = (np.zeros((max(wide_rows, 1), cfg.width), np.float32),
                     np.zeros((max(head_rows, 1), cfg.head_size), np.float32))
        lib().oracle_decoder_capture_norms(self._handle, _p(self._cap[0], ctypes.c_float), wide_rows,
                                           _p(self._cap[1], ctypes.c_float), head_rows)
        return self._cap

    def captured(self):
        """(width-wide rows, head rows) recorded so far."""
        return (self._cap[0][:lib().oracle_decoder_captured(self._handle, 0)],
                self._cap[1][:lib().oracle_decoder_captured(self._handle, 1)])

    def kv(self, layer: int):
        """Copies of the cached K and V rows [position, kv_heads*head_size]."""
        n = self.position * self.config.kv_heads * self.config.head_size
        k = np.ctypeslib.as_array(lib().oracle_decoder_keys(self._handle, layer), shape=(max(n, 1),))[:n].copy()
        v = np.ctypeslib.as_array(lib().oracle_decoder_values(self._handle, layer), shape=(max(n, 1),))[:n].copy()
        return k, v

    def set_kv(self, layer: int, keys: np.ndarray, values: np.ndarray):
        """Overwrite cached rows from position 0 (for long-KV stress inputs)."""
        keys = np.ascontiguousarray(keys, dtype=np.float32).ravel()
        values = np.ascontiguousarray(values, dtype=np.float32).ravel()
        width = self.config.kv_heads * self.config.head_size
        assert keys.size % width == 0 and keys.size // width <= self.capacity
        dst_k = np.ctypeslib.as_array(lib().oracle_decoder_keys(self._handle, layer), shape=(self.capacity * width,))
        dst_v = np.ctypeslib.as_array(lib().oracle_decoder_values(self._handle, layer), shape=(self.capacity * width,))
        dst_k[:keys.size] = keys
        dst_v[:values.size] = values

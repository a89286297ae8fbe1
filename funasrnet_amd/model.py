"""Qwen3 decoder weights: configuration, GGUF mapping and the seeded
synthetic generator used for every measured workload.

Tensor names and metadata keys follow QwenDecoder's constructor
(src/FunAsrNet/QwenDecoder.cs:46-112, 183-267): ``blk.{l}.attn_{q,k,v,output}``,
``ffn_{gate,up,down}``, ``attn_norm``, ``attn_{q,k}_norm``, ``ffn_norm``,
``output_norm``, ``token_embd`` (tied lm_head when ``output.weight`` is absent).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import gguf


@dataclass(frozen=True)
class DecoderConfig:
    width: int = 1024
    heads: int = 16
    kv_heads: int = 8
    head_size: int = 128
    layers: int = 28
    ffn: int = 3072
    vocab: int = 151936
    eps: float = 1e-6
    rope_base: float = 1000000.0

    @property
    def q_width(self) -> int:
        return self.heads * self.head_size

    @property
    def kv_width(self) -> int:
        return self.kv_heads * self.head_size

    def weight_bytes_per_token(self) -> int:
        """Q8_0 bytes streamed per decoded token (34 B per 32 parameters)."""
        per_layer = self.width * (self.q_width + 2 * self.kv_width) + self.q_width * self.width
        per_layer += 3 * self.width * self.ffn
        return (self.layers * per_layer + self.vocab * self.width) * 34 // 32


QWEN3_0_6B = DecoderConfig()


@dataclass
class Q8Tensor:
    """A Q8_0 matrix as the reference holds it after load: int8 [rows, cols]
    row-major and one float32 scale per 32 values [rows, cols/32]. A tensor
    read raw from a GGUF file has ``blocks`` (rows*cols/32 x 34 bytes) and
    ``dims`` instead of the unpacked planes."""

    name: str
    quantized: np.ndarray | None
    scales: np.ndarray | None
    scale_bits: np.ndarray | None = None
    blocks: np.ndarray | None = None
    dims: tuple | None = None  # (rows, cols) when only blocks are held

    @property
    def rows(self) -> int:
        return int(self.quantized.shape[0]) if self.quantized is not None else int(self.dims[0])

    @property
    def columns(self) -> int:
        return int(self.quantized.shape[1]) if self.quantized is not None else int(self.dims[1])


@dataclass
class LayerWeights:
    wq: Q8Tensor
    wk: Q8Tensor
    wv: Q8Tensor
    wo: Q8Tensor
    gate: Q8Tensor
    up: Q8Tensor
    down: Q8Tensor
    attn_norm: np.ndarray
    q_norm: np.ndarray
    k_norm: np.ndarray
    ffn_norm: np.ndarray


@dataclass
class DecoderWeights:
    config: DecoderConfig
    layers: list = field(default_factory=list)
    token_embd: Q8Tensor | None = None
    output: Q8Tensor | None = None  # None: tied to token_embd
    output_norm: np.ndarray | None = None

    @property
    def lm_head(self) -> Q8Tensor:
        return self.output if self.output is not None else self.token_embd


def _q8(rng: np.random.Generator, name: str, rows: int, cols: int) -> Q8Tensor:
    q = rng.integers(-127, 128, size=(rows, cols), dtype=np.int8)
    s = np.abs(rng.standard_normal(rows * cols // 32, dtype=np.float32)) * np.float32(0.02) / np.float32(127.0)
    half = s.astype(np.float16)
    return Q8Tensor(name, q, half.astype(np.float32).reshape(rows, cols // 32), half.view(np.uint16).reshape(rows, cols // 32))


def synthetic(config: DecoderConfig = QWEN3_0_6B, seed: int = 0) -> DecoderWeights:
    """Random-init decoder: int8 ~ U{-127..127}, scales fp16(|N(0,0.02)|/127),
    norm weights 1.0, tied embeddings. numpy PCG64 seeded with ``seed``;
    tensors drawn layer by layer in the order q, k, v, o, gate, up, down,
    then token_embd."""
    rng = np.random.Generator(np.random.PCG64(seed))
    c = config
    w = DecoderWeights(config=c)
    ones = lambda n: np.ones(n, dtype=np.float32)
    for layer in range(c.layers):
        p = f"blk.{layer}."
        w.layers.append(LayerWeights(
            wq=_q8(rng, p + "attn_q.weight", c.q_width, c.width),
            wk=_q8(rng, p + "attn_k.weight", c.kv_width, c.width),
            wv=_q8(rng, p + "attn_v.weight", c.kv_width, c.width),
            wo=_q8(rng, p + "attn_output.weight", c.width, c.q_width),
            gate=_q8(rng, p + "ffn_gate.weight", c.ffn, c.width),
            up=_q8(rng, p + "ffn_up.weight", c.ffn, c.width),
            down=_q8(rng, p + "ffn_down.weight", c.width, c.ffn),
            attn_norm=ones(c.width), q_norm=ones(c.head_size), k_norm=ones(c.head_size), ffn_norm=ones(c.width)))
    w.token_embd = _q8(rng, "token_embd.weight", c.vocab, c.width)
    w.output_norm = ones(c.width)
    return w


def small_config(layers: int = 2, vocab: int = 4096) -> DecoderConfig:
    """A reduced Qwen3-shaped decoder for quick parity runs (head_size 128,
    GQA 2:1 as in the full model)."""
    return DecoderConfig(width=512, heads=4, kv_heads=2, head_size=128, layers=layers, ffn=1024, vocab=vocab)


def to_gguf(weights: DecoderWeights, path: str) -> None:
    c = weights.config
    meta = {
        "general.architecture": "qwen3",
        "qwen3.embedding_length": c.width,
        "qwen3.attention.head_count": c.heads,
        "qwen3.attention.head_count_kv": c.kv_heads,
        "qwen3.attention.key_length": c.head_size,
        "qwen3.block_count": c.layers,
        "qwen3.feed_forward_length": c.ffn,
        "qwen3.attention.layer_norm_rms_epsilon": float(c.eps),
        "qwen3.rope.freq_base": float(c.rope_base),
        # ByteBpe needs these keys (src/FunAsrNet/ByteBpe.cs:33,39); placeholders.
        "tokenizer.ggml.tokens": [f"<t{i}>" for i in range(4)],
        "tokenizer.ggml.merges": ["a b"],
        "tokenizer.ggml.eos_token_id": 151645,
    }

    def q8(t: Q8Tensor):
        bits = t.scale_bits if t.scale_bits is not None else t.scales.astype(np.float16).view(np.uint16)
        return gguf.Weight(t.name, (t.columns, t.rows), quantized=t.quantized.reshape(-1), scales=t.scales.reshape(-1),
                           scale_bits=bits.reshape(-1))

    def f32(name, a):
        return gguf.Weight(name, (a.size,), values=a)

    tensors = []
    for i, L in enumerate(weights.layers):
        p = f"blk.{i}."
        tensors += [q8(L.wq), q8(L.wk), q8(L.wv), q8(L.wo), q8(L.gate), q8(L.up), q8(L.down),
                    f32(p + "attn_norm.weight", L.attn_norm), f32(p + "attn_q_norm.weight", L.q_norm),
                    f32(p + "attn_k_norm.weight", L.k_norm), f32(p + "ffn_norm.weight", L.ffn_norm)]
    tensors.append(q8(weights.token_embd))
    if weights.output is not None:
        tensors.append(q8(weights.output))
    tensors.append(f32("output_norm.weight", weights.output_norm))
    gguf.write(path, meta, tensors)


def from_gguf(model: gguf.Gguf) -> DecoderWeights:
    """QwenDecoder constructor view of a loaded GGUF (QwenDecoder.cs:63-78)."""
    c = DecoderConfig(
        width=model.int("qwen3.embedding_length", 1024),
        heads=model.int("qwen3.attention.head_count", 16),
        kv_heads=model.int("qwen3.attention.head_count_kv", 8),
        head_size=model.int("qwen3.attention.key_length", 128),
        layers=model.int("qwen3.block_count", 28),
        ffn=model["blk.0.ffn_gate.weight"].rows,
        vocab=model["token_embd.weight"].rows,
        eps=model.float("qwen3.attention.layer_norm_rms_epsilon", 1e-6),
        rope_base=model.float("qwen3.rope.freq_base", 1000000.0))
    if c.heads % c.kv_heads != 0:
        raise ValueError("Invalid GQA head counts")

    def q8(name) -> Q8Tensor:
        w = model[name]
        if w.blocks is not None:
            return Q8Tensor(name, None, None, blocks=w.blocks, dims=(w.rows, w.columns))
        if w.quantized is None:
            raise ValueError(f"{name}: decoder projections must be Q8_0")
        return Q8Tensor(name, w.quantized.reshape(w.rows, w.columns), w.scales.reshape(w.rows, w.columns // 32),
                        None if w.scale_bits is None else w.scale_bits.reshape(w.rows, w.columns // 32))

    out = DecoderWeights(config=c)
    for i in range(c.layers):
        p = f"blk.{i}."
        out.layers.append(LayerWeights(
            wq=q8(p + "attn_q.weight"), wk=q8(p + "attn_k.weight"), wv=q8(p + "attn_v.weight"),
            wo=q8(p + "attn_output.weight"), gate=q8(p + "ffn_gate.weight"), up=q8(p + "ffn_up.weight"),
            down=q8(p + "ffn_down.weight"), attn_norm=model[p + "attn_norm.weight"].values,
            q_norm=model[p + "attn_q_norm.weight"].values, k_norm=model[p + "attn_k_norm.weight"].values,
            ffn_norm=model[p + "ffn_norm.weight"].values))
    out.token_embd = q8("token_embd.weight")
    out.output = q8("output.weight") if "output.weight" in model.tensors else None
    out.output_norm = model["output_norm.weight"].values
    return out

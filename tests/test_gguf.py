"""GGUF / Q8_0 model loading (funasrnet_amd/gguf.py) against the reference's
own loading checks, restated (src/FunAsrNet.Checks/Q8ModelLoadingChecks.cs:13-108):
every fp16 scale bit pattern, every payload byte, short-block rejection,
F16 and Q8_0 tensors read back exactly from a hand-written GGUF v3 file,
and a truncated final block rejected."""
import struct

import numpy as np
import pytest

from funasrnet_amd import gguf, model


def _system_half_to_float_bits(bits: np.ndarray) -> np.ndarray:
    """(float)System.Half: exact widening for numbers (numpy's float16 cast),
    and for NaNs the sign, the quiet bit and the payload moved up 13 bits."""
    bits = bits.astype(np.uint16)
    widened = bits.view(np.float16).astype(np.float32).view(np.uint32)
    nan = (bits & 0x7C00) == 0x7C00
    nan &= (bits & 0x3FF) != 0
    quiet = ((bits.astype(np.uint32) & 0x8000) << 16) | 0x7FC00000 | ((bits.astype(np.uint32) & 0x3FF) << 13)
    return np.where(nan, quiet, widened).astype(np.uint32)


def _raw_blocks(blocks: int) -> np.ndarray:
    """Q8ModelLoadingChecks.cs:15-22: scale bits = block index, payload byte
    i of block b = (b*17 + i*31) & 255."""
    raw = np.empty((blocks, 34), dtype=np.uint8)
    b = np.arange(blocks, dtype=np.int64)
    raw[:, 0] = (b & 0xFF).astype(np.uint8)
    raw[:, 1] = ((b >> 8) & 0xFF).astype(np.uint8)
    i = np.arange(32, dtype=np.int64)
    raw[:, 2:] = ((b[:, None] * 17 + i[None, :] * 31) & 255).astype(np.uint8)
    return raw.reshape(-1)


def test_unpack_every_scale_pattern_and_byte():
    blocks = 65536
    raw = _raw_blocks(blocks)
    q, scales, bits = gguf.unpack_q8_0(raw, blocks)
    assert q.dtype == np.int8 and q.size == blocks * 32
    assert np.array_equal(bits, np.arange(blocks, dtype=np.uint16))
    assert np.array_equal(scales.view(np.uint32), _system_half_to_float_bits(np.arange(blocks, dtype=np.uint32)))
    expected = raw.reshape(blocks, 34)[:, 2:].reshape(-1).view(np.int8)
    assert np.array_equal(q, expected)
    # Negative zero and the largest finite half stay exact.
    assert scales[0x8000].view(np.uint32) == 0x80000000
    assert scales[0x7BFF] == np.float32(65504.0)


def test_unpack_rejects_incomplete_block_and_accepts_empty():
    raw = _raw_blocks(1)
    with pytest.raises(ValueError, match="block dimensions"):
        gguf.unpack_q8_0(raw[:33], 1)
    q, s, b = gguf.unpack_q8_0(np.zeros(0, dtype=np.uint8), 0)
    assert q.size == 0 and s.size == 0 and b.size == 0


def _descriptor(name: str, count: int, kind: int, offset: int) -> bytes:
    nb = name.encode()
    return struct.pack("<Q", len(nb)) + nb + struct.pack("<IQIQ", 1, count, kind, offset)


def test_gguf_f16_and_q8_read_back_exactly(tmp_path):
    """Q8ModelLoadingChecks.cs:54-108: a GGUF v3 file written by hand (not by
    gguf.write) with a 65,553-element F16 tensor and a 9,001-block Q8_0 tensor."""
    half_count, q8_blocks = 65553, 9001
    q8 = _raw_blocks(q8_blocks)
    q8_offset = (half_count * 2 + 31) // 32 * 32
    header = struct.pack("<IIQQ", gguf.GGUF_MAGIC, 3, 2, 0)
    header += _descriptor("half", half_count, gguf.TYPE_F16, 0)
    header += _descriptor("q8", q8_blocks * 32, gguf.TYPE_Q8_0, q8_offset)
    start = (len(header) + 31) // 32 * 32
    blob = bytearray(header + b"\0" * (start - len(header)))
    blob += np.arange(half_count, dtype=np.uint32).astype(np.uint16).tobytes()
    blob += b"\0" * (start + q8_offset - len(blob))
    blob += q8.tobytes()
    path = tmp_path / "chunks.gguf"
    path.write_bytes(bytes(blob))

    m = gguf.Gguf.read(str(path))
    half_bits = np.arange(half_count, dtype=np.uint32) & 0xFFFF
    assert np.array_equal(m["half"].values.view(np.uint32), _system_half_to_float_bits(half_bits))
    w = m["q8"]
    assert w.columns == q8_blocks * 32 and w.rows == 1
    assert np.array_equal(w.quantized, q8.reshape(q8_blocks, 34)[:, 2:].reshape(-1).view(np.int8))
    assert np.array_equal(w.scales.view(np.uint32), _system_half_to_float_bits(np.arange(q8_blocks, dtype=np.uint32)))

    path.write_bytes(bytes(blob[:-3]))
    with pytest.raises(EOFError):
        gguf.Gguf.read(str(path))


def test_gguf_rejects_bad_headers(tmp_path):
    path = tmp_path / "bad.gguf"
    path.write_bytes(struct.pack("<IIQQ", 0x12345678, 3, 0, 0))
    with pytest.raises(ValueError, match="Not a GGUF"):
        gguf.Gguf.read(str(path))
    path.write_bytes(struct.pack("<IIQQ", gguf.GGUF_MAGIC, 4, 0, 0))
    with pytest.raises(ValueError, match="version"):
        gguf.Gguf.read(str(path))
    # Unsupported GGML type (Gguf.cs:174-177).
    header = struct.pack("<IIQQ", gguf.GGUF_MAGIC, 3, 1, 0) + _descriptor("t", 32, 2, 0)
    path.write_bytes(header + b"\0" * 64)
    with pytest.raises(ValueError, match="GGML type"):
        gguf.Gguf.read(str(path))


def test_synthetic_model_round_trip(tmp_path):
    """The writer and reader agree on a small synthetic decoder, and the
    embedding row (Weight.CopyRow, Gguf.cs:326-345) is q * scale."""
    cfg = model.small_config(layers=1, vocab=256)
    w = model.synthetic(cfg, seed=2)
    path = tmp_path / "small.gguf"
    model.to_gguf(w, str(path))
    back = gguf.Gguf.read(str(path))
    L = w.layers[0]
    t = back["blk.0.attn_q.weight"]
    assert (t.columns, t.rows) == (cfg.width, cfg.heads * cfg.head_size)
    assert np.array_equal(t.quantized.reshape(L.wq.quantized.shape), L.wq.quantized)
    assert np.array_equal(t.scales.reshape(L.wq.scales.shape).view(np.uint32), L.wq.scales.view(np.uint32))
    emb = back["token_embd.weight"]
    row = emb.copy_row(7)
    q = emb.quantized[7 * cfg.width:8 * cfg.width].astype(np.float64)
    s = np.repeat(emb.scales[7 * cfg.width // 32:8 * cfg.width // 32].astype(np.float64), 32)
    assert np.array_equal(row, (q * s).astype(np.float32))
    assert back.int("qwen3.block_count", 0) == 1


def test_raw_q8_read_keeps_the_file_blocks(tmp_path):
    """Gguf.read(raw_q8=True) returns each Q8_0 tensor's blocks byte for byte
    (for the device-side split); unpacking them gives the default read."""
    cfg = model.small_config(layers=1, vocab=128)
    w = model.synthetic(cfg, seed=4)
    path = tmp_path / "raw.gguf"
    model.to_gguf(w, str(path))
    raw = gguf.Gguf.read(str(path), raw_q8=True)
    full = gguf.Gguf.read(str(path))
    t, u = raw["blk.0.ffn_down.weight"], full["blk.0.ffn_down.weight"]
    assert t.quantized is None and t.blocks.dtype == np.uint8 and t.blocks.size == t.rows * t.columns // 32 * 34
    q, s, bits = gguf.unpack_q8_0(t.blocks, t.blocks.size // 34)
    assert np.array_equal(q, u.quantized) and np.array_equal(s.view(np.uint32), u.scales.view(np.uint32))
    weights = model.from_gguf(raw)
    assert weights.layers[0].down.rows == cfg.width and weights.layers[0].down.columns == cfg.ffn

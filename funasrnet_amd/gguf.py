"""GGUF v2/v3 reader and writer with the reference's tensor semantics.

Mirrors ``Gguf`` and ``Weight`` (src/FunAsrNet/Gguf.cs:10-345) and
``UnpackQ8Model`` (src/FunAsrNet/TensorMath.Q8Model.cs:15-39): GGML
dimension order (``columns = shape[0]``, ``rows = shape[1]``), F32 and F16
tensors widened to float32, Q8_0 34-byte blocks unpacked into a row-major
int8 plane plus one float32 scale per 32 values. Any other GGML type is
rejected, as the reference does (Gguf.cs:174-177).

This is load-time host code; it never runs on the decode path.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

GGUF_MAGIC = 0x46554747
TYPE_F32, TYPE_F16, TYPE_Q8_0 = 0, 1, 8
_BLOCK = 34


def half_bits_to_float(bits: np.ndarray) -> np.ndarray:
    """Exact binary16 -> binary32 widening; NaNs come back quiet with their
    payload shifted up, as System.Half's explicit float conversion does."""
    h = np.asarray(bits, dtype=np.uint16).astype(np.uint32)
    sign = (h & 0x8000) << 16
    exponent = (h >> 10) & 0x1F
    mantissa = h & 0x3FF
    normal = sign | ((exponent + 112) << 23) | (mantissa << 13)
    special = np.where(mantissa == 0, sign | 0x7F800000, sign | 0x7FC00000 | (mantissa << 13))
    sub = (mantissa.astype(np.float32) * np.float32(2.0 ** -24)).view(np.uint32) | sign
    out = np.where(exponent == 0, sub, np.where(exponent == 31, special, normal))
    return out.astype(np.uint32).view(np.float32)


def unpack_q8_0(raw: np.ndarray, blocks: int):
    """TensorMath.UnpackQ8Model: little-endian fp16 scale, then 32 int8."""
    raw = np.asarray(raw, dtype=np.uint8)
    if raw.size != blocks * _BLOCK:
        raise ValueError("Q8 model block dimensions differ")
    b = raw.reshape(blocks, _BLOCK)
    bits = b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8)
    return b[:, 2:].copy().view(np.int8).reshape(-1), half_bits_to_float(bits), bits


def pack_q8_0(quantized: np.ndarray, scale_bits: np.ndarray) -> bytes:
    q = np.ascontiguousarray(quantized, dtype=np.int8).reshape(-1, 32)
    bits = np.ascontiguousarray(scale_bits, dtype=np.uint16).reshape(-1)
    out = np.empty((q.shape[0], _BLOCK), dtype=np.uint8)
    out[:, 0] = (bits & 0xFF).astype(np.uint8)
    out[:, 1] = (bits >> 8).astype(np.uint8)
    out[:, 2:] = q.view(np.uint8)
    return out.tobytes()


@dataclass
class Weight:
    """Gguf.cs:264-345. ``shape`` is in GGML order (innermost first)."""

    name: str
    shape: tuple
    values: np.ndarray | None = None      # float32, F32/F16 tensors
    quantized: np.ndarray | None = None   # int8 [rows * columns]
    scales: np.ndarray | None = None      # float32 [rows * columns / 32]
    scale_bits: np.ndarray | None = None  # raw fp16 bits, kept for re-writing
    blocks: np.ndarray | None = None      # raw Q8_0 blocks (34 B each), when read with raw_q8

    @property
    def columns(self) -> int:
        return int(self.shape[0])

    @property
    def rows(self) -> int:
        return int(self.shape[1]) if len(self.shape) > 1 else 1

    def copy_row(self, index: int) -> np.ndarray:
        """Weight.CopyRow (Gguf.cs:326-345): q[j] * scale[j/32] for Q8_0."""
        c = self.columns
        if self.values is not None:
            return self.values[index * c:(index + 1) * c].copy()
        q = self.quantized[index * c:(index + 1) * c].astype(np.float32)
        s = np.repeat(self.scales[index * c // 32:(index + 1) * c // 32], 32)
        return (q * s).astype(np.float32)


class _Reader:
    def __init__(self, data: memoryview):
        self.data = data
        self.pos = 0

    def take(self, n: int) -> memoryview:
        if self.pos + n > len(self.data):
            raise EOFError("truncated GGUF")
        v = self.data[self.pos:self.pos + n]
        self.pos += n
        return v

    def unpack(self, fmt: str):
        size = struct.calcsize(fmt)
        return struct.unpack("<" + fmt, self.take(size))[0]

    def string(self) -> str:
        n = self.unpack("Q")
        if n > 64 * 1024 * 1024:
            raise ValueError("Oversized GGUF string")
        return bytes(self.take(n)).decode("utf-8")

    def value(self, kind: int):
        scalar = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}
        if kind in scalar:
            return self.unpack(scalar[kind])
        if kind == 8:
            return self.string()
        if kind == 9:
            inner = self.unpack("I")
            n = self.unpack("Q")
            return [self.value(inner) for _ in range(n)]
        raise ValueError(f"Unknown GGUF metadata type {kind}")


@dataclass
class Gguf:
    """Gguf.cs:43-185: metadata plus tensors by name."""

    metadata: dict = field(default_factory=dict)
    tensors: dict = field(default_factory=dict)

    def int(self, key: str, fallback: int) -> int:
        return int(self.metadata[key]) if key in self.metadata else fallback

    def float(self, key: str, fallback: float) -> float:
        return float(np.float32(self.metadata[key])) if key in self.metadata else fallback

    def __getitem__(self, key: str) -> Weight:
        return self.tensors[key]

    @classmethod
    def read(cls, path: str, raw_q8: bool = False) -> "Gguf":
        """Read a GGUF file. With ``raw_q8`` the Q8_0 tensors keep their
        34-byte blocks as they are in the file (``Weight.blocks``) instead
        of being unpacked, for uploads that split them on the device."""
        with open(path, "rb") as f:
            data = memoryview(f.read())
        r = _Reader(data)
        if r.unpack("I") != GGUF_MAGIC:
            raise ValueError("Not a GGUF model")
        version = r.unpack("I")
        if version not in (2, 3):
            raise ValueError(f"GGUF version {version}")
        tensor_count, metadata_count = r.unpack("Q"), r.unpack("Q")
        model = cls()
        for _ in range(metadata_count):
            key = r.string()
            if key in model.metadata:
                raise ValueError(f"duplicate metadata key {key}")
            model.metadata[key] = r.value(r.unpack("I"))
        descriptors = []
        for _ in range(tensor_count):
            name = r.string()
            dims = r.unpack("I")
            if not 1 <= dims <= 4:
                raise ValueError("Invalid tensor rank")
            shape = tuple(r.unpack("Q") for _ in range(dims))
            descriptors.append((name, shape, r.unpack("I"), r.unpack("Q")))
        alignment = model.int("general.alignment", 32)
        if alignment <= 0:
            raise ValueError("Invalid alignment")
        start = (r.pos + alignment - 1) // alignment * alignment
        for name, shape, kind, offset in descriptors:
            count = int(np.prod(shape))
            at = start + offset
            w = Weight(name, shape)
            if kind == TYPE_F32:
                w.values = _slice(data, at, count * 4).view(np.float32).copy()
            elif kind == TYPE_F16:
                w.values = half_bits_to_float(_slice(data, at, count * 2).view(np.uint16))
            elif kind == TYPE_Q8_0:
                if shape[0] % 32 != 0:
                    raise ValueError("Q8_0 row not aligned")
                blocks = count // 32
                if raw_q8:
                    w.blocks = _slice(data, at, blocks * _BLOCK).copy()
                else:
                    w.quantized, w.scales, w.scale_bits = unpack_q8_0(_slice(data, at, blocks * _BLOCK), blocks)
            else:
                raise ValueError(f"Tensor {name}: GGML type {kind}")
            if name in model.tensors:
                raise ValueError(f"duplicate tensor {name}")
            model.tensors[name] = w
        return model


def _slice(data: memoryview, at: int, n: int) -> np.ndarray:
    if at < 0 or at + n > len(data):
        raise EOFError("truncated GGUF tensor data")
    return np.frombuffer(data[at:at + n], dtype=np.uint8)


def _encode_value(value) -> bytes:
    if isinstance(value, bool):
        return struct.pack("<I?", 7, value)
    if isinstance(value, int):
        return struct.pack("<Ii", 5, value) if -2**31 <= value < 2**31 else struct.pack("<Iq", 11, value)
    if isinstance(value, float):
        return struct.pack("<If", 6, value)
    if isinstance(value, str):
        b = value.encode("utf-8")
        return struct.pack("<IQ", 8, len(b)) + b
    if isinstance(value, (list, tuple)):
        if all(isinstance(v, str) for v in value):
            body = b"".join(struct.pack("<Q", len(v.encode())) + v.encode() for v in value)
            return struct.pack("<IIQ", 9, 8, len(value)) + body
        if all(isinstance(v, int) for v in value):
            return struct.pack("<IIQ", 9, 5, len(value)) + struct.pack(f"<{len(value)}i", *value)
    raise TypeError(f"unsupported metadata value {value!r}")


def write(path: str, metadata: dict, tensors: list[Weight], alignment: int = 32) -> None:
    """Write a GGUF v3 file (F32, F16 values, or Q8_0 with raw scale bits)."""
    header = bytearray()
    header += struct.pack("<IIQQ", GGUF_MAGIC, 3, len(tensors), len(metadata))
    for key, value in metadata.items():
        kb = key.encode()
        header += struct.pack("<Q", len(kb)) + kb + _encode_value(value)
    payloads = []
    offset = 0
    for w in tensors:
        if w.quantized is not None:
            kind, blob = TYPE_Q8_0, pack_q8_0(w.quantized, w.scale_bits)
        else:
            kind, blob = TYPE_F32, np.ascontiguousarray(w.values, dtype=np.float32).tobytes()
        nb = w.name.encode()
        header += struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(w.shape))
        header += b"".join(struct.pack("<Q", d) for d in w.shape)
        header += struct.pack("<IQ", kind, offset)
        payloads.append((offset, blob))
        offset = (offset + len(blob) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(header)
        start = (len(header) + alignment - 1) // alignment * alignment
        f.write(b"\0" * (start - len(header)))
        pos = 0
        for off, blob in payloads:
            f.write(b"\0" * (off - pos))
            f.write(blob)
            pos = off + len(blob)

"""A minimal GGUF v2/v3 reader for test fixtures.

Follows the layout the reference's reader parses (src/tensomite/gguf.cr:297-376):
magic, version, tensor and metadata counts, typed metadata values, tensor
infos (name, dims innermost first, kind, offset), then the data section at
the next multiple of `general.alignment` (32 by default). Shapes are returned
outermost first, as tensomite reports them. Reads data only; executes nothing.
"""
from __future__ import annotations

import struct

import numpy as np

MAGIC = 0x46554747
KIND_NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 8: "Q8_0", 30: "BF16"}
BLOCK_BYTES = {"Q4_0": 18, "Q4_1": 20, "Q8_0": 34}


class GGUF:
    def __init__(self, path: str):
        with open(path, "rb") as f:
            self.data = f.read()
        self.pos = 0
        if self._u32() != MAGIC:
            raise ValueError(f"{path} is not a GGUF file")
        version = self._u32()
        if version not in (2, 3):
            raise ValueError(f"GGUF version {version} is not supported")
        tensors, keys = self._u64(), self._u64()
        self.metadata = {}
        for _ in range(keys):
            key = self._string()
            self.metadata[key] = self._value(self._u32())
        infos = []
        for _ in range(tensors):
            name = self._string()
            dims = [self._u64() for _ in range(self._u32())]
            kind = self._u32()
            offset = self._u64()
            infos.append((name, list(reversed(dims)), kind, offset))
        alignment = int(self.metadata.get("general.alignment", 32))
        start = (self.pos + alignment - 1) // alignment * alignment
        self.entries = {}
        for name, shape, kind, offset in infos:
            self.entries[name] = (KIND_NAMES[kind], shape, start + offset)

    def _take(self, n: int) -> bytes:
        out = self.data[self.pos:self.pos + n]
        self.pos += n
        return out

    def _u32(self) -> int:
        return struct.unpack("<I", self._take(4))[0]

    def _u64(self) -> int:
        return struct.unpack("<Q", self._take(8))[0]

    def _string(self) -> str:
        return self._take(self._u64()).decode("utf-8")

    def _value(self, kind: int):
        fmt = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
        if kind in fmt:
            size = struct.calcsize(fmt[kind])
            return struct.unpack(fmt[kind], self._take(size))[0]
        if kind == 8:
            return self._string()
        if kind == 9:
            element = self._u32()
            return [self._value(element) for _ in range(self._u64())]
        raise ValueError(f"GGUF value type {kind} is not known")

    def kind(self, name: str) -> str:
        return self.entries[name][0]

    def shape(self, name: str) -> list:
        return self.entries[name][1]

    def raw(self, name: str) -> np.ndarray:
        """The tensor's bytes as stored (block bytes for Q formats)."""
        kind, shape, offset = self.entries[name]
        count = int(np.prod(shape))
        if kind in BLOCK_BYTES:
            size = count // 32 * BLOCK_BYTES[kind]
        else:
            size = count * (4 if kind == "F32" else 2)
        return np.frombuffer(self.data, dtype=np.uint8, count=size, offset=offset).copy()

    def f32(self, name: str) -> np.ndarray:
        kind, shape, offset = self.entries[name]
        if kind != "F32":
            raise ValueError(f"{name} is {kind}")
        return self.raw(name).view(np.float32).reshape(shape)


def write(path: str, metadata, tensors, alignment: int = 32) -> None:
    """Writes a GGUF v3 file: metadata as (key, value) pairs (int -> uint32
    or int64, float -> float32, str, bool), tensors as (name, kind name or
    ggml code, shape outermost first, bytes) in that order, data aligned as
    the reader expects (gguf.cr:156-191's layout)."""
    codes = {v: k for k, v in KIND_NAMES.items()}
    out = bytearray()
    out += struct.pack("<IIQQ", MAGIC, 3, len(tensors), len(metadata))

    def string(s):
        b = s.encode()
        return struct.pack("<Q", len(b)) + b

    for key, value in metadata:
        out += string(key)
        if isinstance(value, bool):
            out += struct.pack("<IB", 7, value)
        elif isinstance(value, int):
            out += struct.pack("<II", 4, value) if 0 <= value < 2 ** 32 else struct.pack("<Iq", 11, value)
        elif isinstance(value, float):
            out += struct.pack("<If", 6, value)
        else:
            out += struct.pack("<I", 8) + string(value)
    offset = 0
    offsets = []
    for name, kind, shape, data in tensors:
        offsets.append(offset)
        out += string(name) + struct.pack("<I", len(shape))
        for d in reversed(shape):
            out += struct.pack("<Q", d)
        out += struct.pack("<IQ", codes.get(kind, kind), offset)
        offset += (len(data) + alignment - 1) // alignment * alignment
    out += b"\0" * ((-len(out)) % alignment)
    for (name, kind, shape, data), off in zip(tensors, offsets):
        out += bytes(data)
        out += b"\0" * ((-len(out)) % alignment)
    with open(path, "wb") as f:
        f.write(out)

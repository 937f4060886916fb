"""A GGUF v3 writer for tests: the llama.cpp container layout (little-endian
header, typed metadata, tensor infos with ne in fastest-axis-first order,
data section at `general.alignment`), as the reference's own reader tests
build their images (src/gguf/reader.rs:397-430)."""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STRING:
        return _str(v)
    if vtype == ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[vtype], v)


def write(path, metadata: list, tensors: list, alignment: int = 32) -> None:
    """metadata: [(key, vtype, value)]; tensors: [(name, torch_shape, ggml_type, data bytes)].
    Tensor data is laid out in order, each start aligned."""
    out = bytearray()
    out += struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(metadata))
    for k, t, v in metadata:
        out += _str(k) + struct.pack("<I", t) + _value(t, v)
    offs, off = [], 0
    for _, _, _, data in tensors:
        offs.append(off)
        off += len(data)
        off = (off + alignment - 1) // alignment * alignment
    for (name, shape, gtype, _), o in zip(tensors, offs):
        ne = list(reversed(shape))
        out += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        out += struct.pack("<IQ", gtype, o)
    out += b"\0" * ((-len(out)) % alignment)
    base = len(out)
    for (_, _, _, data), o in zip(tensors, offs):
        out += b"\0" * (base + o - len(out))
        out += bytes(np.asarray(data, dtype=np.uint8).tobytes())
    with open(path, "wb") as f:
        f.write(out)

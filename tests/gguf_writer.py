"""A minimal GGUF (v2/v3, little-endian) file writer for tests. TEST
INFRASTRUCTURE ONLY.

Layout, from the published GGUF format: the magic "GGUF", u32 version, u64
tensor count, u64 key/value count; each key/value pair as a string key
(u64 length + bytes), a u32 value type and the value (arrays: u32 element
type, u64 count, elements); each tensor's info as its name (string), u32
dimension count, u64 dimensions (innermost first), u32 ggml type and u64
offset from the start of the data section; then padding to the alignment
(general.alignment, 32 by default) and the data section, in which every
tensor starts at a multiple of the alignment.
"""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STRING:
        return _str(v)
    if vtype == ARRAY:
        etype, items = v
        return struct.pack("<IQ", etype, len(items)) + b"".join(_value(etype, e) for e in items)
    return struct.pack(_SCALAR[vtype], v)


def write_gguf(path: str, kvs: list, tensors: list, alignment: int = 32,
               version: int = 3) -> dict:
    """kvs: [(key, vtype, value)]; tensors: [(name, ggml_type, dims, data)]
    with dims innermost first and data the encoded bytes (np.uint8 array).
    A general.alignment entry in kvs must agree with `alignment`. Returns
    {name: offset of the tensor's bytes from the start of the file}."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    head += b"".join(_str(k) + struct.pack("<I", t) + _value(t, v) for k, t, v in kvs)
    offsets, off = [], 0
    for _, _, _, data in tensors:
        offsets.append(off)
        off += -(-len(data) // alignment) * alignment
    for (name, gtype, dims, _), o in zip(tensors, offsets):
        head += _str(name) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", gtype, o)
    data_start = -(-len(head) // alignment) * alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * (data_start - len(head)))
        for (_, _, _, data), o in zip(tensors, offsets):
            f.write(np.ascontiguousarray(data, dtype=np.uint8).tobytes())
            f.write(b"\0" * (-len(data) % alignment))
    return {name: data_start + o for (name, _, _, _), o in zip(tensors, offsets)}

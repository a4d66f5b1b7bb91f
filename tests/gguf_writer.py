"""Writes GGUF v3 files for the loader tests, from the public container format: magic,
version 3, counts, typed key-value pairs, tensor infos (dims with the row length first,
ggml type, offset in the data region), padding to the alignment, the data region."""
import struct

import numpy as np

_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    if t == 8:
        return _str(v)
    if t == 9:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for it in items:
            out += _str(it) if et == 8 else struct.pack(_SCALAR[et], it)
        return out
    return struct.pack(_SCALAR[t], v)


def write_gguf(path, kvs, tensors, alignment=32):
    """kvs: [(key, type, value)]; tensors: [(name, dims, ggml_type, raw bytes)].  Tensor
    data is laid out in order, each at a multiple of the alignment."""
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kvs))
    for key, t, v in kvs:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    data, offs = b"", []
    for _, _, _, raw in tensors:
        pad = (-len(data)) % alignment
        data += b"\0" * pad
        offs.append(len(data))
        data += bytes(raw)
    for (name, dims, typ, _), off in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", typ, off)
    head += b"\0" * ((-len(head)) % alignment)
    with open(path, "wb") as f:
        f.write(head + data)
    return len(head), offs

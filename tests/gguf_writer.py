"""Minimal GGUF (version 3) writer for loader tests (test infrastructure): key-values and tensors with their data,
laid out as the container defines (header, key-values, tensor infos, data section at general.alignment)."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
GGML_F32, GGML_F16, GGML_I8, GGML_I16 = 0, 1, 24, 25
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STR:
        return _str(v)
    if t == ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for it in items:
            out += _value(et, it)
        return out
    return struct.pack(_SCALAR[t], v)


def write(path, kvs, tensors, alignment=32):
    """kvs: [(key, type, value)]; tensors: [(name, ggml_type, ne list, raw bytes)] (raw is written as given)"""
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kvs)))
    for k, t, v in kvs:
        out += _str(k) + struct.pack("<I", t) + _value(t, v)
    offs, off = [], 0
    for name, gt, ne, raw in tensors:
        offs.append(off)
        off += (len(raw) + alignment - 1) // alignment * alignment
    for (name, gt, ne, raw), o in zip(tensors, offs):
        out += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", e) for e in ne) + struct.pack("<IQ", gt, o)
    out += b"\0" * ((-len(out)) % alignment)
    for (name, gt, ne, raw), o in zip(tensors, offs):
        out += bytes(raw)
        out += b"\0" * ((-len(out)) % alignment)
    with open(path, "wb") as f:
        f.write(out)


def as_bytes(a):
    return np.ascontiguousarray(a).tobytes()

"""Writes GGUF files for the loader tests (the public GGUF v3 layout that
barq_core/src/gguf.rs:250-337 reads: little-endian, u64 counts and string
lengths, typed KV values, tensor infos, aligned data section)."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}


def _string(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(t, v) -> bytes:
    if t == STRING:
        return _string(v)
    if t == ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[t], int(v) if t == BOOL else v)


def write(path, kvs, tensors, alignment=None, version=3, magic=b"GGUF", truncate=0):
    """kvs: [(key, type, value)]; tensors: [(name, dims, type_id, raw bytes)].
    Tensor data is laid out in order, each at a multiple of the alignment."""
    al = alignment if alignment is not None else 32
    head = magic + struct.pack("<IQQ", version, len(tensors), len(kvs))
    head += b"".join(_string(k) + struct.pack("<I", t) + _value(t, v) for k, t, v in kvs)
    offsets, off = [], 0
    for _, _, _, raw in tensors:
        offsets.append(off)
        off = (off + len(raw) + al - 1) // al * al
    for (name, dims, tid, raw), o in zip(tensors, offsets):
        head += _string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", tid, o)
    data_offset = (len(head) + al - 1) // al * al
    blob = bytearray(head + b"\0" * (data_offset - len(head)))
    for (name, dims, tid, raw), o in zip(tensors, offsets):
        end = data_offset + o
        blob += b"\0" * (end - len(blob))
        blob += bytes(raw)
    if truncate:
        blob = blob[:-truncate]
    with open(path, "wb") as f:
        f.write(bytes(blob))
    return data_offset, offsets

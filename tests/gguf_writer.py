"""Minimal GGUF v3 writer for the tests, written from the public GGUF layout description: magic
"GGUF", u32 version, u64 tensor count, u64 kv count, kv pairs (u64-length string key, u32 value
type, value), tensor infos (name, u32 n_dims, u64 dims, u32 ggml type, u64 offset relative to the
data section), zero padding to the alignment, tensor data (each tensor aligned). Little-endian."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _val(t, v):
    if t == STR:
        return _str(v)
    if t == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_val(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def write(path, kv, tensors, alignment=32, version=3):
    """kv: [(key, type, value)]; tensors: [(name, dims, ggml_type, raw bytes)]. Returns the absolute
    data offsets of the tensors."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv))
    for k, t, v in kv:
        head += _str(k) + struct.pack("<I", t) + _val(t, v)
    tensors = [(n, d, t, np.ascontiguousarray(r, dtype=np.uint8).reshape(-1)) for n, d, t, r in tensors]
    rel, off = [], 0
    for name, dims, ty, raw in tensors:
        off = -(-off // alignment) * alignment
        rel.append(off)
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ty, off)
        off += len(raw)
    start = -(-len(head) // alignment) * alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * (start - len(head)))
        pos = 0
        for (name, dims, ty, raw), r in zip(tensors, rel):
            f.write(b"\0" * (r - pos))
            f.write(raw.tobytes())
            pos = r + len(raw)
    return [start + r for r in rel]

"""A small GGUF v3 writer for test fixtures (test infrastructure).

Writes the layout ggml's gguf_write_to_file produces (ggml/src/gguf.cpp,
gguf_write_out 1622-1660): header, KV pairs in insertion order, tensor infos,
padding to the alignment, tensor data each padded to the alignment with zeros.
tests/golden/gen_gguf.py checks, where the reference build exists, that the
files written here are byte-identical to the ones the reference writer produces
for the same content, and records their SHA-256 for the GPU box.
"""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}
# ggml type -> (elements per block, bytes per block) for the types the fixtures use
GGML_BLOCK = {0: (1, 4), 1: (1, 2), 8: (32, 34), 12: (256, 144), 14: (256, 210)}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    if t == STRING:
        return _str(v)
    return struct.pack(_FMT[t], v)


def kv_bytes(key: str, t: int, v, arr_type: int | None = None) -> bytes:
    out = _str(key) + struct.pack("<i", t)
    if t == ARRAY:
        out += struct.pack("<iQ", arr_type, len(v))
        for x in v:
            out += _value(arr_type, x)
    else:
        out += _value(t, v)
    return out


def tensor_nbytes(ggml_type: int, ne) -> int:
    blck, size = GGML_BLOCK[ggml_type]
    n = int(np.prod(ne, dtype=np.int64))
    return n // blck * size


def write_gguf(path, kvs, tensors, alignment: int = 32, version: int = 3) -> bytes:
    """kvs: [(key, type, value[, array element type])]; tensors: [(name, ggml_type,
    ne (list, ne0 first), data bytes)].  Returns the bytes written."""
    pad = lambda n: (n + alignment - 1) // alignment * alignment  # noqa: E731
    head = b"GGUF" + struct.pack("<Iqq", version, len(tensors), len(kvs))
    for kv in kvs:
        head += kv_bytes(kv[0], kv[1], kv[2], kv[3] if len(kv) > 3 else None)
    off = 0
    infos = b""
    for name, t, ne, data in tensors:
        assert len(data) == tensor_nbytes(t, ne)
        infos += _str(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}q", *ne)
        infos += struct.pack("<iQ", t, off)
        off += pad(len(data))
    meta = head + infos
    out = bytearray(meta + b"\0" * (pad(len(meta)) - len(meta)))
    for _, _, _, data in tensors:
        out += data + b"\0" * (pad(len(data)) - len(data))
    with open(path, "wb") as f:
        f.write(out)
    return bytes(out)

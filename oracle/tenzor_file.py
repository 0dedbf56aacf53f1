"""TEST INFRASTRUCTURE ONLY — pure-Python restatement of the .tenzor format
(io/tenzor_format.zig): hashName, TenzorWriter.finish, TenzorFile.open +
getTensor, convertFromSafetensors.

Only tests/ may import this module; it is the checker, never shipped.

Pinning (tests/test_tenzor_format.py): the reference's own tests
(tenzor_format.zig:490-575: header and entry sizes, hash equal/unequal,
dtype sizes, write-and-read of two f32 tensors, numel of a 3-D entry),
published FNV-1a 64-bit test vectors, and round trips through the
independent safetensors library.
"""
from __future__ import annotations

import struct

PAGE = 4096
MAGIC = b"TENZOR\x00\x00"
HEADER = struct.Struct("<8sIIIIQQI20s")          # tenzor_format.zig:66-80
ENTRY = struct.Struct("<QBB2x5IQQ")              # tenzor_format.zig:83-92
DTYPE_SIZE = [4, 2, 2, 8, 1, 2, 4, 8, 1, 2, 4, 8]  # byteSize, tenzor_format.zig:39-46
# safetensors dtype names -> tenzor_format.DType (tenzor_format.zig:454-468)
FROM_ST = {"F32": 0, "F16": 1, "BF16": 2, "F64": 3, "I8": 4, "I16": 5, "I32": 6, "I64": 7, "U8": 8, "U16": 9,
           "U32": 10, "U64": 11, "BOOL": 8}


def hash_name(name: bytes) -> int:
    h = 0xcbf29ce484222325
    for c in name:
        h = ((h ^ c) * 0x100000001b3) & 0xFFFFFFFFFFFFFFFF
    return h


def _up(v, a):
    return (v + a - 1) & ~(a - 1)


def write(tensors, metadata: bytes = b"{}") -> bytes:
    """TenzorWriter.finish (tenzor_format.zig:352-428); tensors are
    (name bytes, dtype, shape tuple, data bytes) in order."""
    index_offset = HEADER.size + _up(len(metadata), 8)
    data_offset = _up(index_offset + len(tensors) * ENTRY.size, PAGE)
    out = bytearray(HEADER.pack(MAGIC, 1, 0, len(tensors), 0, index_offset, data_offset, len(metadata), b"\0" * 20))
    out += metadata + b"\0" * (_up(len(metadata), 8) - len(metadata))
    off = 0
    for name, dtype, shape, data in tensors:
        dims = list(shape[:5]) + [0] * (5 - min(len(shape), 5))
        out += ENTRY.pack(hash_name(name), dtype, len(shape), *dims, off, len(data))
        off += len(data)
    out += b"\0" * (data_offset - len(out))
    for _, _, _, data in tensors:
        out += data
    return bytes(out)


def read(blob: bytes):
    """TenzorFile.open (tenzor_format.zig:140-197): (metadata, entries) with
    entries as dicts, each carrying its data bytes."""
    magic, version, _flags, count, _pad, index_offset, data_offset, meta_size, _ = HEADER.unpack_from(blob, 0)
    if magic != MAGIC:
        raise ValueError("InvalidMagic")
    if version != 1:
        raise ValueError("UnsupportedVersion")
    meta = blob[HEADER.size:HEADER.size + meta_size]
    entries = []
    for i in range(count):
        h, dt, nd, *rest = ENTRY.unpack_from(blob, index_offset + i * ENTRY.size)
        dims, doff, dsize = rest[:5], rest[5], rest[6]
        entries.append(dict(hash=h, dtype=dt, ndim=nd, shape=tuple(dims[:nd]), data=blob[data_offset + doff:
                                                                                         data_offset + doff + dsize]))
    return meta, entries


def get(entries, name: bytes):
    """getTensorByHash without a name map: the first entry with the hash."""
    h = hash_name(name)
    return next((e for e in entries if e["hash"] == h), None)


def convert_safetensors(st_bytes: bytes) -> bytes:
    """convertFromSafetensors (tenzor_format.zig:440-484): every tensor in
    header order, metadata "{}"."""
    import json

    n = struct.unpack_from("<Q", st_bytes, 0)[0]
    header = json.loads(st_bytes[8:8 + n])  # json keeps the file's key order
    base = 8 + n
    tensors = []
    for name, info in header.items():
        if name == "__metadata__":
            continue
        s, e = info["data_offsets"]
        tensors.append((name.encode(), FROM_ST[info["dtype"]], tuple(info["shape"]), st_bytes[base + s:base + e]))
    return write(tensors)

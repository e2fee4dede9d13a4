"""Minimal GGUF writer for the tests (test infrastructure, not shipped).

Writes the container format the reference parses (swamp-gguf/src/mmap.rs:34-94,
metadata.rs:117-243), following the published GGUF layout:

    magic "GGUF" | u32 version | n_tensors | n_kv        (u32 counts in v1, u64 after)
    n_kv x (string key, u32 type, value)
    n_tensors x (string name, u32 n_dims, dims (u32 in v1, u64 after),
                 u32 dtype, u64 offset relative to the data section)
    zero padding to a multiple of `align`, then the tensor data

Strings are u64 length + bytes.  Arrays are u32 element type + u64 count +
elements.  Everything is little-endian.  Independent of the C reader under
test, so a round trip pins the reader.
"""
from __future__ import annotations

import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}


def _string(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STRING:
        return _string(v)
    if vtype == ARRAY:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(_value(etype, e) for e in items)
    return struct.pack(_SCALAR[vtype], v)


def write_gguf(path, tensors, kv=(), version=3, align=32, tail=b"", magic=b"GGUF",
               raw_kv=b"", truncate=None):
    """tensors: list of (name, shape, dtype, data_bytes[, offset]); offsets
    default to consecutive, each aligned to `align`.  kv: list of
    (key, type, value).  Returns (data_offset, [absolute offsets])."""
    wide = version >= 2
    cnt = "<Q" if wide else "<I"
    head = bytearray(magic + struct.pack("<I", version))
    head += struct.pack(cnt, len(tensors)) + struct.pack(cnt, len(kv) + (1 if raw_kv else 0))
    for key, vtype, val in kv:
        head += _string(key) + struct.pack("<I", vtype) + _value(vtype, val)
    head += raw_kv
    rel, cur = [], 0
    for t in tensors:
        if len(t) > 4:
            rel.append(t[4])
        else:
            cur = (cur + align - 1) // align * align
            rel.append(cur)
            cur += len(t[3])
    for (name, shape, dtype, data, *_), off in zip(tensors, rel):
        head += _string(name) + struct.pack("<I", len(shape))
        for d in shape:
            head += struct.pack("<Q" if wide else "<I", d)
        head += struct.pack("<IQ", dtype, off)
    data_offset = (len(head) + align - 1) // align * align
    blob = bytearray(head) + bytes(data_offset - len(head))
    for (name, shape, dtype, data, *_), off in zip(tensors, rel):
        end = data_offset + off + len(data)
        if len(blob) < end:
            blob += bytes(end - len(blob))
        blob[data_offset + off:end] = data
    blob += tail
    if truncate is not None:
        blob = blob[:truncate]
    with open(path, "wb") as f:
        f.write(blob)
    return data_offset, [data_offset + o for o in rel]

"""A GGUF v2/v3 writer for the tests, written from the container's published layout:

  magic "GGUF" | version u32 | tensor count u64 | key/value count u64
  key/value: key (u64 length + bytes) | value type u32 | value
  tensor info: name | n_dims u32 | dims u64 x n_dims (innermost first) | type u32 | offset u64
  padding to the alignment (32), then the data section; offsets are relative to it.

Value types: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool, 8 string, 9 array
(element type u32 + count u64 + elements), 10 u64, 11 i64, 12 f64.
"""
from __future__ import annotations

import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
        U64: "<Q", I64: "<q", F64: "<d"}


def _str(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STR:
        return _str(v)
    if vtype == ARR:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        for it in items:
            out += _value(etype, it)
        return out
    return struct.pack(_FMT[vtype], v)


def write_gguf(path, kv, tensors, version=3, align=32, pad_data=0):
    """kv: list of (key, value type, value); tensors: list of (name, dims rows-first,
    ggml type, raw bytes). Tensor data is laid out in order, each at a multiple of align.
    Returns the list of (name, offset) and the data section's file offset."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv))
    for key, vt, v in kv:
        head += _str(key) + struct.pack("<I", vt) + _value(vt, v)
    offsets, off = [], 0
    for name, dims, gtype, raw in tensors:
        offsets.append((name, off))
        off += len(raw)
        off = (off + align - 1) // align * align
    for (name, dims, gtype, raw), (_, o) in zip(tensors, offsets):
        head += _str(name) + struct.pack("<I", len(dims))
        for d in reversed(dims):
            head += struct.pack("<Q", d)
        head += struct.pack("<IQ", gtype, o)
    data_at = (len(head) + align - 1) // align * align
    body = bytearray(head + b"\0" * (data_at - len(head)))
    for (name, dims, gtype, raw), (_, o) in zip(tensors, offsets):
        need = data_at + o + len(raw)
        if len(body) < data_at + o:
            body += b"\0" * (data_at + o - len(body))
        body[data_at + o: need] = raw
    body += b"\0" * pad_data
    with open(path, "wb") as f:
        f.write(body)
    return offsets, data_at

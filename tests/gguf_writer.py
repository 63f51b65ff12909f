"""Minimal GGUF v3 writer for tests: well-formed files, and the raw pieces to build malformed
ones.  Layout per the format src/gguf.rs:95-179 reads: magic, version, tensor count,
metadata count, metadata (key, type, value), tensor infos (name, rank, dims, kind, offset),
padding to the alignment, tensor data.
"""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
        U64: "<Q", I64: "<q", F64: "<d"}


def gstr(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def value(t: int, v) -> bytes:
    if t == STR:
        return gstr(v)
    if t == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(value(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def kv(key: str, t: int, v) -> bytes:
    return gstr(key) + struct.pack("<I", t) + value(t, v)


def tensor_info(name: str, dims, kind: int, offset: int) -> bytes:
    return gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) + \
        struct.pack("<IQ", kind, offset)


def header(nt: int, nk: int, version: int = 3, magic: bytes = b"GGUF") -> bytes:
    return magic + struct.pack("<IQQ", version, nt, nk)


def build(meta: list[tuple[str, int, object]], tensors: list[tuple[str, list[int], int, bytes]],
          align: int = 32) -> bytes:
    """A well-formed GGUF: meta = [(key, type, value)], tensors = [(name, dims, kind, raw)]."""
    out = bytearray(header(len(tensors), len(meta)))
    for k, t, v in meta:
        out += kv(k, t, v)
    offs, off = [], 0
    for _, _, _, raw in tensors:
        offs.append(off)
        off += len(raw)
        off = (off + align - 1) // align * align
    for (name, dims, kind, _), o in zip(tensors, offs):
        out += tensor_info(name, dims, kind, o)
    out += b"\0" * ((-len(out)) % align)
    base = len(out)
    for (_, _, _, raw), o in zip(tensors, offs):
        out += b"\0" * (base + o - len(out))
        out += raw
    return bytes(out)


def f32_bytes(a) -> bytes:
    return np.ascontiguousarray(np.asarray(a, dtype="<f4")).tobytes()


def f16_bytes(a) -> bytes:
    return np.ascontiguousarray(np.asarray(a, dtype="<f2")).tobytes()

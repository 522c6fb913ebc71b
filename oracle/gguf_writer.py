"""Minimal GGUF v3 writer — test infrastructure only.

Writes the synthetic model files that the compiled reference (oracle/_ref)
loads to produce golden vectors and the reference CPU baseline, and the
files the GGUF reader tests open.  The layout follows the GGUF container as
the reference parses it (gguf.c:289-404): magic, version, tensor_count,
metadata_count, metadata (key, type, value), tensor infos (name, n_dims,
dims[], type, offset), then the data section aligned to general.alignment
(default 32).
"""
from __future__ import annotations

import struct

import numpy as np

GGUF_UINT32, GGUF_FLOAT32, GGUF_STRING, GGUF_ARRAY = 4, 6, 8, 9

# metadata kind -> (gguf value type, struct format); "str" and "arr" apart
KINDS = {"u8": (0, "<B"), "i8": (1, "<b"), "u16": (2, "<H"), "i16": (3, "<h"),
         "u32": (4, "<I"), "i32": (5, "<i"), "f32": (6, "<f"), "bool": (7, "<B"),
         "str": (8, None), "arr": (9, None), "u64": (10, "<Q"), "i64": (11, "<q"),
         "f64": (12, "<d")}


def _str(s) -> bytes:
    b = s if isinstance(s, (bytes, bytearray)) else s.encode()
    return struct.pack("<Q", len(b)) + bytes(b)


def _bytes(raw) -> memoryview:
    """Raw little-endian bytes of a bytes object or numpy array."""
    if isinstance(raw, (bytes, bytearray)):
        return memoryview(raw)
    return memoryview(np.ascontiguousarray(raw).reshape(-1).view(np.uint8))


def _value(kind, val) -> bytes:
    """Type tag + payload of one metadata value.  kind "arr" takes
    val = (elem_kind, list); elem_kind "arr" nests (elem_kind, list) pairs."""
    t, fmt = KINDS[kind]
    return struct.pack("<I", t) + _payload(kind, val)


def _payload(kind, val) -> bytes:
    t, fmt = KINDS[kind]
    if kind == "str":
        return _str(val)
    if kind == "arr":
        ek, items = val
        out = struct.pack("<I", KINDS[ek][0]) + struct.pack("<Q", len(items))
        return out + b"".join(_payload(ek, v) for v in items)
    if kind == "bool":
        return struct.pack(fmt, 1 if val else 0)
    if kind in ("f32", "f64"):
        return struct.pack(fmt, float(val))
    return struct.pack(fmt, int(val))


def gguf_bytes(metadata, tensors, alignment: int = 32, version: int = 3,
               with_data: bool = True) -> bytes:
    """The file as bytes.  metadata: list of (key, kind, value), kinds as in
    KINDS.  tensors: list of (name, ggml_type, dims, raw_bytes); raw_bytes
    may be None for a tensor info without data (then with_data should be
    False, as in the reference's header-only test files).  Tensors are laid
    out in list order, each at the next multiple of `alignment`."""
    head = bytearray()
    head += b"GGUF"
    head += struct.pack("<I", version)
    head += struct.pack("<Q", len(tensors))
    head += struct.pack("<Q", len(metadata))
    for key, kind, val in metadata:
        head += _str(key) + _value(kind, val)
    blobs = [_bytes(raw) if raw is not None else memoryview(b"") for _, _, _, raw in tensors]
    offsets = []
    off = 0
    for (_, _, _, raw), blob in zip(tensors, blobs):
        off = (off + alignment - 1) // alignment * alignment
        offsets.append(off)
        off += len(blob)
    for (name, typ, dims, _), o in zip(tensors, offsets):
        head += _str(name)
        head += struct.pack("<I", len(dims))
        for d in dims:
            head += struct.pack("<Q", int(d))
        head += struct.pack("<I", int(typ))
        head += struct.pack("<Q", o)
    if not with_data:
        return bytes(head)
    out = bytearray(head)
    out += b"\0" * ((-len(head)) % alignment)
    base = len(out)
    for blob, o in zip(blobs, offsets):
        out += b"\0" * (base + o - len(out))
        out += blob
    return bytes(out)


def write_gguf(path: str, metadata, tensors, alignment: int = 32, version: int = 3,
               with_data: bool = True) -> None:
    """Write gguf_bytes(...) to `path`."""
    with open(path, "wb") as f:
        f.write(gguf_bytes(metadata, tensors, alignment, version, with_data))

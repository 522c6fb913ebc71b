"""Minimal GGUF v3 writer — test infrastructure only.

Writes the synthetic model files that the compiled reference (oracle/_ref)
loads to produce golden vectors and the reference CPU baseline.  The layout
follows the GGUF container as the reference parses it (gguf.c:289-404):
magic, version, tensor_count, metadata_count, metadata (key, type, value),
tensor infos (name, n_dims, dims[], type, offset), then the data section
aligned to general.alignment (default 32).
"""
from __future__ import annotations

import struct

import numpy as np

GGUF_UINT32, GGUF_FLOAT32, GGUF_STRING = 4, 6, 8


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _bytes(raw) -> memoryview:
    """Raw little-endian bytes of a bytes object or numpy array."""
    if isinstance(raw, (bytes, bytearray)):
        return memoryview(raw)
    return memoryview(np.ascontiguousarray(raw).reshape(-1).view(np.uint8))


def write_gguf(path: str, metadata, tensors, alignment: int = 32) -> None:
    """metadata: list of (key, kind, value) with kind in {'u32','f32','str'}.
    tensors: list of (name, ggml_type, dims, raw_bytes)."""
    head = bytearray()
    head += b"GGUF"
    head += struct.pack("<I", 3)
    head += struct.pack("<Q", len(tensors))
    head += struct.pack("<Q", len(metadata))
    for key, kind, val in metadata:
        head += _str(key)
        if kind == "u32":
            head += struct.pack("<I", GGUF_UINT32) + struct.pack("<I", int(val))
        elif kind == "f32":
            head += struct.pack("<I", GGUF_FLOAT32) + struct.pack("<f", float(val))
        elif kind == "str":
            head += struct.pack("<I", GGUF_STRING) + _str(str(val))
        else:
            raise ValueError(kind)
    blobs = [_bytes(raw) for _, _, _, raw in tensors]
    offsets = []
    off = 0
    for blob in blobs:
        off = (off + alignment - 1) // alignment * alignment
        offsets.append(off)
        off += len(blob)
    for (name, typ, dims, raw), o in zip(tensors, offsets):
        head += _str(name)
        head += struct.pack("<I", len(dims))
        for d in dims:
            head += struct.pack("<Q", int(d))
        head += struct.pack("<I", int(typ))
        head += struct.pack("<Q", o)
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * pad)
        pos = 0
        for blob, o in zip(blobs, offsets):
            if o > pos:
                f.write(b"\0" * (o - pos))
                pos = o
            f.write(blob)
            pos += len(blob)

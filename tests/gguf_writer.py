"""A small GGUF v3 writer for the loader tests (test infrastructure).

Writes the container as the GGUF format defines it: the magic and version,
tensor and key counts, key/value metadata, tensor descriptors (name, GGML-order
shape, type, offset into the data section), then the data section at the
header's end rounded up to the alignment, each tensor at an aligned offset.
Options produce the malformed files the error tests need.
"""
from __future__ import annotations

import struct

import numpy as np

# GGUF value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
           I64: "<q", F64: "<d"}

# GGML type -> (elements per block, bytes per block)
BLOCKS = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144), 14: (256, 210), 24: (1, 1), 30: (1, 2)}


def _string(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, value) -> bytes:
    if vtype == STRING:
        return _string(value)
    if vtype == ARRAY:
        etype, items = value
        return struct.pack("<IQ", etype, len(items)) + b"".join(_value(etype, v) for v in items)
    return struct.pack(_SCALAR[vtype], value)


def tensor_bytes(ggml_type: int, shape) -> int:
    e, b = BLOCKS[ggml_type]
    n = int(np.prod(shape))
    return n // e * b


def write(path, metadata=(), tensors=(), alignment: int = 32, magic: bytes = b"GGUF", version: int = 3,
          truncate: int | None = None, extra_tensor_bytes: int = 0):
    """metadata: (key, value type, value) triples; arrays as (element type, [items]).
    tensors: (name, GGML-order shape, GGML type, raw bytes). Returns the data
    section's offset."""
    header = bytearray()
    header += magic + struct.pack("<IQQ", version, len(tensors), len(metadata))
    for key, vtype, value in metadata:
        header += _string(key) + struct.pack("<I", vtype) + _value(vtype, value)
    offsets, at = [], 0
    for name, shape, gtype, data in tensors:
        at = (at + alignment - 1) // alignment * alignment
        offsets.append(at)
        at += len(data)
    for (name, shape, gtype, data), off in zip(tensors, offsets):
        header += _string(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        header += struct.pack("<IQ", gtype, off)
    start = (len(header) + alignment - 1) // alignment * alignment
    body = bytearray(header) + bytes(start - len(header))
    for (name, shape, gtype, data), off in zip(tensors, offsets):
        body += bytes(start + off - len(body))
        body += bytes(data)
    body += bytes(extra_tensor_bytes)
    if truncate is not None:
        body = body[:truncate]
    with open(path, "wb") as f:
        f.write(body)
    return start

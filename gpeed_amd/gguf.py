"""GGUF v3 file writer for fixtures and tools.

Writes the layout ggml defines and the reference parses (cpp/core/src/gguf.cpp:
135-187). The arrangement follows python/tools/make_test_gguf.py:126-205:
- magic, version, tensor count, key/value count;
- the key/value pairs;
- the tensor infos (name, dims in ggml order, type id, data offset);
- zero padding to the alignment;
- the tensor data, each payload starting on an alignment boundary relative
  to the start of the data section.

This is a writer of its own; the reference's script is not used. Values take
every GGUF value type, arrays (nested too) included.
"""
from __future__ import annotations

import struct
from typing import Iterable, Sequence

import numpy as np

# value types (GGUF spec; cpp/core/include/glm5/gguf.h:15-29)
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
           BOOL: "<B", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}

# tensor types used by the tests (ggml ids) and their geometry: (elements per
# block, bytes per block)
F32, F16, Q8_0, Q6_K, IQ3_XXS, IQ4_XS, BF16 = 0, 1, 8, 14, 18, 23, 30
GEOMETRY = {0: (1, 4), 1: (1, 2), 30: (1, 2), 8: (32, 34), 2: (32, 18), 10: (256, 84), 11: (256, 110),
            14: (256, 210), 18: (256, 98), 21: (256, 110), 22: (256, 82), 23: (256, 136), 24: (1, 1),
            26: (1, 4)}


def row_bytes(dtype: int, n: int) -> int:
    bs, ts = GEOMETRY[dtype]
    if n % bs:
        raise ValueError(f"{n} elements are not whole blocks of {bs}")
    return n // bs * ts


def _str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STRING:
        return _str(v)
    if vtype == ARRAY:
        etype, items = v
        return struct.pack("<IQ", etype, len(items)) + b"".join(_value(etype, x) for x in items)
    if vtype == BOOL:
        return struct.pack("<B", 1 if v else 0)
    return struct.pack(_SCALAR[vtype], v)


def encode(kvs: Sequence[tuple], tensors: Sequence[tuple], version: int = 3) -> bytes:
    """The file's bytes.

    kvs: (key, value_type, value); an ARRAY value is (element_type, items).
    tensors: (name, dims in ggml order, type id, payload as bytes or uint8 array).
    The alignment is the value of a "general.alignment" key, else 32.
    """
    alignment = 32
    for k, vt, v in kvs:
        if k == "general.alignment":
            alignment = int(v)
    head = bytearray(b"GGUF")
    head += struct.pack("<IQQ", version, len(tensors), len(kvs))
    for k, vt, v in kvs:
        head += _str(k) + struct.pack("<I", vt) + _value(vt, v)
    data = bytearray()
    infos = []
    for name, dims, dtype, payload in tensors:
        raw = bytes(np.ascontiguousarray(payload).view(np.uint8).reshape(-1)) if not isinstance(payload, bytes) \
            else payload
        data += b"\0" * (-len(data) % alignment)
        infos.append((name, list(dims), dtype, len(data)))
        data += raw
    for name, dims, dtype, off in infos:
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", dtype, off)
    head += b"\0" * (-len(head) % alignment)
    return bytes(head) + bytes(data)


def write(path: str, kvs: Sequence[tuple], tensors: Sequence[tuple], version: int = 3) -> dict:
    """Writes the file; returns {tensor name: (offset in the data section, byte count)}."""
    blob = encode(kvs, tensors, version)
    with open(path, "wb") as f:
        f.write(blob)
    return layout(kvs, tensors)


def layout(kvs: Sequence[tuple], tensors: Iterable[tuple]) -> dict:
    alignment = next((int(v) for k, vt, v in kvs if k == "general.alignment"), 32)
    out, pos = {}, 0
    for name, dims, dtype, payload in tensors:
        n = len(payload) if isinstance(payload, bytes) else np.asarray(payload).nbytes
        pos += -pos % alignment
        out[name] = (pos, n)
        pos += n
    return out

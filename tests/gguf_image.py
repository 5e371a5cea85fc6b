"""Writer of small GGUF images for the tests (GGUF v2/v3 layout: header,
metadata key/values, tensor table, data section aligned to `alignment`)."""
from __future__ import annotations

import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
        BOOL: "<B", U64: "<Q", I64: "<q", F64: "<d"}


def _str(s) -> bytes:
    b = s if isinstance(s, bytes) else s.encode()
    return struct.pack("<Q", len(b)) + b


def _scalar(t: int, v) -> bytes:
    return _str(v) if t == STR else struct.pack(_FMT[t], v)


def value(t: int, v, elem_type: int = 0) -> bytes:
    """Typed metadata value; for ARR, v is the list and elem_type its type."""
    if t == ARR:
        return (struct.pack("<IIQ", ARR, elem_type, len(v)) +
                b"".join(_scalar(elem_type, e) for e in v))
    return struct.pack("<I", t) + _scalar(t, v)


def image(metadata=(), tensors=(), version: int = 3, alignment: int = 32,
          offsets=None) -> bytes:
    """metadata: [(key, encoded value bytes)]; tensors: [(name, dims, ggml type,
    payload bytes)].  Payloads go into the data section, each at an offset
    rounded up to `alignment` (or at the given relative offsets)."""
    out = struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(metadata))
    for key, enc in metadata:
        out += _str(key) + enc
    rel, pos = [], 0
    for i, (_, _, _, payload) in enumerate(tensors):
        pos = (pos + alignment - 1) // alignment * alignment
        rel.append(offsets[i] if offsets is not None else pos)
        pos += len(payload)
    for (name, dims, ty, _), off in zip(tensors, rel):
        out += _str(name) + struct.pack("<I", len(dims))
        out += b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", ty, off)
    data_start = (len(out) + alignment - 1) // alignment * alignment
    out += b"\0" * (data_start - len(out))
    data = bytearray(max([o + len(t[3]) for o, t in zip(rel, tensors)], default=0))
    for (_, _, _, payload), off in zip(tensors, rel):
        data[off:off + len(payload)] = payload
    return out + bytes(data)

"""GGUF header parsing restated from the reference -- TEST INFRASTRUCTURE ONLY.

Pure Python (``struct``), the checker for the library's GGUF parser.  Each
function follows crates/realm-core/src/formats/gguf.rs:
  parse_header          gguf.rs:111-160 (magic, version 2..3, counts)
  read_metadata_value   gguf.rs:367-400 (value types 0..12, arrays)
  read_typed_value      gguf.rs:402-425 (array elements; no nested arrays)
  parse_tensor_info     gguf.rs:427-455 (name, n_dims, u64 dims, type, offset)
  tensor_data_offset    gguf.rs:165-175 (end of the table rounded up to 32)
  as_u32 / as_f32       gguf.rs:50-71
  extract_config        gguf.rs:212-280 (keys, fallback keys, defaults)
  Shape::validate       crates/realm-core/src/tensor.rs:102-110
Errors are raised as GgufError with the ErrorCode the reference's Error maps
to (crates/realm-runtime/src/lib.rs:122-134): 4 ParseError/InvalidFormat,
7 Io (read_exact past the end), 3 InvalidShape.
"""
from __future__ import annotations

import struct

GGUF_MAGIC = 0x46554747
INVALID_ARGUMENT, MODEL_PARSE_ERROR, IO_ERROR = 3, 4, 7
# value type -> struct format of its scalar (8 = string, 9 = array)
SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B",
          10: "<Q", 11: "<q", 12: "<d"}
INT_TYPES = (0, 1, 2, 3, 4, 5, 10, 11)


class GgufError(Exception):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


class _Reader:
    def __init__(self, data: bytes):
        self.d, self.pos = data, 0

    def take(self, n: int) -> bytes:
        if self.pos + n > len(self.d):
            raise GgufError(IO_ERROR, "failed to fill whole buffer")
        b = self.d[self.pos:self.pos + n]
        self.pos += n
        return b

    def fmt(self, f: str):
        return struct.unpack(f, self.take(struct.calcsize(f)))[0]

    def string(self) -> str:
        n = self.fmt("<Q")
        raw = self.take(n)
        try:
            return raw.decode("utf-8")
        except UnicodeDecodeError as e:
            raise GgufError(MODEL_PARSE_ERROR, f"Invalid UTF-8: {e}")


def _typed(r: _Reader, t: int):
    if t == 8:
        return (8, r.string())
    if t in SCALAR:
        v = r.fmt(SCALAR[t])
        return (t, bool(v) if t == 7 else v)
    raise GgufError(MODEL_PARSE_ERROR, f"Unknown typed value: {t}")


def _value(r: _Reader):
    t = r.fmt("<I")
    if t == 9:
        et = r.fmt("<I")
        n = r.fmt("<Q")
        return (9, [_typed(r, et) for _ in range(n)])
    if t == 8 or t in SCALAR:
        return _typed(r, t)
    raise GgufError(MODEL_PARSE_ERROR, f"Unknown metadata value type: {t}")


def parse(data: bytes) -> dict:
    """{'version', 'tensor_count', 'kv_count', 'metadata': {key: (type, value)},
    'tensors': [(name, dims, type, offset)], 'data_offset'}"""
    r = _Reader(data)
    magic = r.fmt("<I")
    if magic != GGUF_MAGIC:
        raise GgufError(MODEL_PARSE_ERROR, f"Invalid GGUF magic: 0x{magic:08X}")
    version = r.fmt("<I")
    if not 2 <= version <= 3:
        raise GgufError(MODEL_PARSE_ERROR, f"Unsupported GGUF version: {version}")
    tensor_count = r.fmt("<Q")
    kv_count = r.fmt("<Q")
    metadata = {}
    for _ in range(kv_count):
        key = r.string()
        metadata[key] = _value(r)
    tensors = []
    for _ in range(tensor_count):
        name = r.string()
        nd = r.fmt("<I")
        dims = tuple(r.fmt("<Q") for _ in range(nd))
        ty = r.fmt("<I")
        off = r.fmt("<Q")
        if not dims:
            raise GgufError(INVALID_ARGUMENT, "Shape cannot be empty")
        if 0 in dims:
            raise GgufError(INVALID_ARGUMENT, "Shape dimensions must be > 0")
        tensors.append((name, dims, ty, off))
    data_offset = (r.pos + 31) & ~31
    return {"version": version, "tensor_count": tensor_count, "kv_count": kv_count,
            "metadata": metadata, "tensors": tensors, "data_offset": data_offset}


def as_u32(v):
    if v is None or v[0] not in INT_TYPES:
        return None
    return v[1] & 0xFFFFFFFF


def as_f32(v):
    if v is None or v[0] not in (6, 12):
        return None
    return struct.unpack("<f", struct.pack("<f", v[1]))[0]


def extract_config(meta: dict) -> dict:
    md = meta["metadata"]
    a = md.get("general.architecture")
    arch = a[1] if a is not None and a[0] == 8 else "unknown"

    def get(k1, k2, conv, default):
        v = md.get(k1)
        if v is None:
            v = md.get(k2)
        out = conv(v)
        return default if out is None else out

    return {
        "vocab_size": get(f"{arch}.vocab_size", "vocab_size", as_u32, 32000),
        "hidden_size": get(f"{arch}.embedding_length", f"{arch}.hidden_size", as_u32, 2048),
        "num_layers": get(f"{arch}.block_count", f"{arch}.num_layers", as_u32, 22),
        "num_heads": get(f"{arch}.attention.head_count", f"{arch}.num_heads", as_u32, 32),
        "num_kv_heads": get(f"{arch}.attention.head_count_kv", f"{arch}.num_kv_heads", as_u32, 4),
        "intermediate_size": get(f"{arch}.feed_forward_length", f"{arch}.intermediate_size",
                                 as_u32, 5632),
        "max_seq_len": get(f"{arch}.context_length", f"{arch}.max_seq_len", as_u32, 2048),
        "rms_norm_eps": get(f"{arch}.attention.layer_norm_rms_epsilon", "rms_norm_eps", as_f32,
                            struct.unpack("<f", struct.pack("<f", 1e-5))[0]),
        "rope_theta": get(f"{arch}.rope.freq_base", "rope_theta", as_f32, 10000.0),
    }

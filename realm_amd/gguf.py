"""GGUF model images through librealm_hip: the mirror of the reference's
``GGUFParser`` (crates/realm-core/src/formats/gguf.rs:111-280) and of
ModelStorage's tensor table (crates/realm-runtime/src/model_storage.rs:
386-487), with the image's quantized 2-D tensors registered once as resident
device weights.

Parsing runs in the library on the host and needs no GPU; ``register``
needs the device (a ``HipGpuBackend`` initialised first).  Errors raise the
same ``RealmError`` classes as the backend, with the reference's ErrorCode
values: 4 for a malformed image, 7 for an image that ends inside the header,
3 for an invalid tensor shape.
"""
from __future__ import annotations

import ctypes
from ctypes import byref, c_int, c_size_t, c_uint32, c_uint64, c_void_p
from typing import NamedTuple

import numpy as np

from . import _lib
from .backend import _ERRORS, RealmError


class TensorDesc(NamedTuple):
    """One entry of the tensor table (TensorDesc, crates/realm-core/src/tensor.rs:113-130)."""
    name: str
    ggml_type: int
    dims: tuple          # ggml order: dims[0] is the row length
    offset: int          # absolute byte offset in the image
    nbytes: int          # 0 for types the library does not size


class RealmGgufConfig(ctypes.Structure):
    _fields_ = [("vocab_size", c_uint32), ("hidden_size", c_uint32), ("num_layers", c_uint32),
                ("num_heads", c_uint32), ("num_kv_heads", c_uint32),
                ("intermediate_size", c_uint32), ("max_seq_len", c_uint32),
                ("rms_norm_eps", ctypes.c_float), ("rope_theta", ctypes.c_float)]


class GgufModel:
    """A parsed GGUF image (the bytes ModelStorage::store_model receives)."""

    def __init__(self, image):
        self.lib = _lib.load()
        self.image = np.frombuffer(bytes(image), dtype=np.uint8)
        h = c_uint64()
        self._check(self.lib.realm_hip_gguf_parse(self._ptr(), self.image.size, byref(h)))
        self.handle = h.value
        v, tc, kc, do = c_uint32(), c_uint64(), c_uint64(), c_uint64()
        self._check(self.lib.realm_hip_gguf_info(self.handle, byref(v), byref(tc), byref(kc),
                                                 byref(do)))
        self.version, self.tensor_count = v.value, tc.value
        self.metadata_kv_count, self.data_offset = kc.value, do.value

    def _ptr(self) -> c_void_p:
        return c_void_p(self.image.ctypes.data) if self.image.size else c_void_p(0)

    def _check(self, rc: int) -> None:
        if rc != 0:
            raise _ERRORS.get(rc, RealmError)(rc, self.lib.realm_hip_last_error().decode())

    # ------------------------------------------------------------ table
    def tensor(self, index: int) -> TensorDesc:
        name = ctypes.create_string_buffer(4096)
        t, nd, off, nb = c_int(), c_uint32(), c_uint64(), c_uint64()
        dims = (c_uint64 * 4)()
        self._check(self.lib.realm_hip_gguf_tensor(self.handle, index, name, len(name), byref(t),
                                                   byref(nd), dims, byref(off), byref(nb)))
        return TensorDesc(name.value.decode(), t.value, tuple(dims[:min(nd.value, 4)]),
                          off.value, nb.value)

    def tensors(self) -> list:
        return [self.tensor(i) for i in range(self.tensor_count)]

    def find(self, name: str) -> int:
        i = c_size_t()
        self._check(self.lib.realm_hip_gguf_find(self.handle, name.encode(), byref(i)))
        return i.value

    # --------------------------------------------------------- metadata
    def meta_u32(self, key: str):
        """MetadataValue::as_u32 of `key`, or None."""
        v = c_uint32()
        rc = self.lib.realm_hip_gguf_meta_u32(self.handle, key.encode(), byref(v))
        return v.value if rc == 0 else None

    def meta_str(self, key: str):
        """MetadataValue::as_string of `key`, or None."""
        buf = ctypes.create_string_buffer(1 << 16)
        rc = self.lib.realm_hip_gguf_meta_str(self.handle, key.encode(), buf, len(buf))
        return buf.value.decode() if rc == 0 else None

    def extract_config(self) -> dict:
        """GGUFParser::extract_config (gguf.rs:212-280)."""
        c = RealmGgufConfig()
        self._check(self.lib.realm_hip_gguf_config(self.handle, byref(c)))
        return {name: getattr(c, name) for name, _ in RealmGgufConfig._fields_}

    # ------------------------------------------------------------ device
    def register(self) -> int:
        """Upload every 2-D Q4_K / Q6_K / Q8_0 tensor once; returns how many."""
        n = c_size_t()
        self._check(self.lib.realm_hip_gguf_register(self.handle, self._ptr(), self.image.size,
                                                     byref(n)))
        return n.value

    def weight(self, name: str):
        """(weight handle, n rows, k row length) of a registered tensor."""
        h, n, k = c_uint64(), c_size_t(), c_size_t()
        self._check(self.lib.realm_hip_gguf_weight(self.handle, name.encode(), byref(h),
                                                   byref(n), byref(k)))
        return h.value, n.value, k.value

    def release(self) -> None:
        if self.handle:
            h, self.handle = self.handle, 0
            self._check(self.lib.realm_hip_gguf_release(h))


__all__ = ["GgufModel", "TensorDesc"]

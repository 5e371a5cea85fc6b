"""Python mirror of Realm's GpuBackendTrait over the HIP C ABI.

``HipGpuBackend`` exposes the trait's method names and argument meaning
(crates/realm-compute-gpu/src/gpu_backend_trait.rs:17-143): ``matmul(a, b, m,
k, n)`` and ``fused_dequant_matmul_{q4k,q6k,q80}(blocks, input, batch_size, n,
k)``, returning an owned f32 array of ``batch_size * n`` elements or raising
``RealmError`` (the ``realm_core::Error`` of crates/realm-core/src/error.rs:4-34,
mapped from the C ABI's ErrorCode).  The trait's other fused formats raise
``BackendError`` so a dispatcher falls back to the CPU, as
crates/realm-models/src/matmul_dispatch.rs:72-88 does on any Err.

Beyond the trait: GPU dequantization, device-resident weights, multi-tenant
LoRA, the candle_matmul host-function surface, and device-buffer plumbing.
"""
from __future__ import annotations

import ctypes
from ctypes import byref, c_float, c_int, c_size_t, c_uint64, c_void_p

import numpy as np

from . import _lib
from .formats import DTYPES, GGML_Q4_K, GGML_Q6_K, GGML_Q8_0

OK, GENERIC_FAILURE, OUT_OF_MEMORY, INVALID_ARGUMENT = 0, 1, 2, 3
MODEL_PARSE_ERROR, BACKEND_UNSUPPORTED = 4, 5
DTYPE_F32, DTYPE_F16 = 0, 1


class RealmError(RuntimeError):
    """A non-zero realm_status; ``code`` is the ErrorCode value."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


class InvalidShape(RealmError):
    pass


class BackendError(RealmError):
    pass


_ERRORS = {INVALID_ARGUMENT: InvalidShape, BACKEND_UNSUPPORTED: BackendError}


def _ptr(a: np.ndarray | None) -> c_void_p:
    return c_void_p(0 if a is None else a.ctypes.data)


class DeviceBuffer:
    """A device allocation owned by the HIP library (freed on close)."""

    def __init__(self, backend: "HipGpuBackend", nbytes: int):
        self._b = backend
        p = c_void_p()
        backend._check(backend.lib.realm_hip_malloc(byref(p), nbytes))
        self.ptr = p.value
        self.nbytes = nbytes

    def upload(self, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        self._b._check(self._b.lib.realm_hip_memcpy_htod(c_void_p(self.ptr), _ptr(a), a.nbytes))
        return self

    def download(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype)
        assert out.nbytes <= self.nbytes
        self._b._check(self._b.lib.realm_hip_memcpy_dtoh(_ptr(out), c_void_p(self.ptr), out.nbytes))
        return out

    def close(self) -> None:
        if self.ptr:
            self._b._check(self._b.lib.realm_hip_free(c_void_p(self.ptr)))
            self.ptr = None

    def __del__(self):  # best effort
        try:
            self.close()
        except Exception:
            pass


class HipGpuBackend:
    """GpuBackendTrait implemented on gfx950 through librealm_hip.so."""

    def __init__(self, device: int = 0):
        self.lib = _lib.load()
        self._check(self.lib.realm_hip_init(device))

    # ------------------------------------------------------------ errors
    def last_error(self) -> str:
        return self.lib.realm_hip_last_error().decode()

    def _check(self, rc: int) -> None:
        if rc != OK:
            raise _ERRORS.get(rc, RealmError)(rc, self.last_error())

    # ----------------------------------------------------- trait methods
    def name(self) -> str:
        return self.lib.realm_hip_backend_name().decode()

    def last_kernel(self) -> str:
        """Name of the last kernel this thread launched (diagnostic)."""
        return self.lib.realm_hip_last_kernel().decode()

    def matmul(self, a, b, m: int, k: int, n: int) -> np.ndarray:
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        out = np.empty(m * n, np.float32)
        self._check(self.lib.realm_hip_matmul(_ptr(a), a.size, _ptr(b), b.size, m, k, n,
                                              _ptr(out)))
        return out

    def dense_matmul_dev(self, d_a: int, d_b: int, d_c: int, m: int, k: int, n: int,
                         transposed: bool = False, stream=None) -> None:
        """C = A @ B (B [k,n]) or A @ B^T (B [n,k]) on device pointers."""
        self._check(self.lib.realm_hip_matmul_dev(c_void_p(d_a), c_void_p(d_b), c_void_p(d_c),
                                                  m, k, n, 1 if transposed else 0,
                                                  c_void_p(stream or 0)))

    def _fused(self, ggml_type: int, blocks, input, batch_size: int, n: int, k: int):
        blocks = np.ascontiguousarray(blocks)
        if blocks.dtype != DTYPES[ggml_type]:
            blocks = blocks.view(DTYPES[ggml_type])
        x = np.ascontiguousarray(input, np.float32)
        out = np.empty(batch_size * n, np.float32)
        self._check(self.lib.realm_hip_fused_dequant_matmul(
            ggml_type, _ptr(blocks), blocks.size, _ptr(x), x.size, batch_size, n, k, _ptr(out)))
        return out

    def fused_dequant_matmul_q4k(self, blocks, input, batch_size, n, k):
        return self._fused(GGML_Q4_K, blocks, input, batch_size, n, k)

    def fused_dequant_matmul_q6k(self, blocks, input, batch_size, n, k):
        return self._fused(GGML_Q6_K, blocks, input, batch_size, n, k)

    def fused_dequant_matmul_q80(self, blocks, input, batch_size, n, k):
        return self._fused(GGML_Q8_0, blocks, input, batch_size, n, k)

    # bytes per block of the formats passed as raw bytes: the reference's
    # 32-element formats (quant.rs:10-70) and its own 256-element Q5_K,
    # Q8_K, Q2_K, Q3_K layouts (quant.rs:71-95, 200-222)
    BLOCK32_BYTES = {"q40": 18, "q41": 20, "q50": 22, "q51": 24, "q81": 36,
                     "q5k": 178, "q8k": 292, "q2k": 116, "q3k": 196}

    def _fused_raw(self, fmt: str, blocks, input, batch_size: int, n: int, k: int):
        """Blocks of the formats above as raw bytes (or a record array)."""
        raw = np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
        x = np.ascontiguousarray(input, np.float32)
        out = np.empty(batch_size * n, np.float32)
        fn = getattr(self.lib, f"realm_hip_fused_dequant_matmul_{fmt}")
        self._check(fn(_ptr(raw), raw.size // self.BLOCK32_BYTES[fmt], _ptr(x), x.size,
                       batch_size, n, k, _ptr(out)))
        return out

    def fused_dequant_matmul_q5k(self, blocks, input, batch_size, n, k):
        return self._fused_raw("q5k", blocks, input, batch_size, n, k)

    def fused_dequant_matmul_q8k(self, blocks, input, batch_size, n, k):
        return self._fused_raw("q8k", blocks, input, batch_size, n, k)

    def fused_dequant_matmul_q2k(self, blocks, input, batch_size, n, k):
        return self._fused_raw("q2k", blocks, input, batch_size, n, k)

    def fused_dequant_matmul_q3k(self, blocks, input, batch_size, n, k):
        return self._fused_raw("q3k", blocks, input, batch_size, n, k)

    def fused_dequant_matmul_q40(self, blocks, input, batch_size, n, k):
        return self._fused_raw("q40", blocks, input, batch_size, n, k)

    def fused_dequant_matmul_q41(self, blocks, input, batch_size, n, k):
        return self._fused_raw("q41", blocks, input, batch_size, n, k)

    def fused_dequant_matmul_q50(self, blocks, input, batch_size, n, k):
        return self._fused_raw("q50", blocks, input, batch_size, n, k)

    def fused_dequant_matmul_q51(self, blocks, input, batch_size, n, k):
        return self._fused_raw("q51", blocks, input, batch_size, n, k)

    def fused_dequant_matmul_q81(self, blocks, input, batch_size, n, k):
        return self._fused_raw("q81", blocks, input, batch_size, n, k)

    # ------------------------------------------------------------ extras
    def set_nan_fallback(self, enable: bool) -> None:
        self._check(self.lib.realm_hip_set_nan_fallback(1 if enable else 0))

    def dequantize(self, ggml_type: int, data, element_count: int) -> np.ndarray:
        raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        out = np.empty(element_count, np.float32)
        self._check(self.lib.realm_hip_dequantize(ggml_type, _ptr(raw), raw.size,
                                                  element_count, _ptr(out)))
        return out

    def candle_matmul(self, mem: np.ndarray, a_ptr, b_ptr, result_ptr, m, k, n,
                      transposed=False) -> int:
        assert mem.dtype == np.uint8 and mem.flags.c_contiguous
        fn = (self.lib.realm_hip_candle_matmul_transposed if transposed
              else self.lib.realm_hip_candle_matmul)
        return fn(_ptr(mem), mem.size, a_ptr, b_ptr, result_ptr, m, k, n)

    def register_weights(self, ggml_type: int, blocks, n: int, k: int) -> int:
        raw = np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
        h = c_uint64()
        self._check(self.lib.realm_hip_weights_register(ggml_type, _ptr(raw), raw.size, n, k,
                                                        byref(h)))
        return h.value

    def release_weights(self, handle: int) -> None:
        self._check(self.lib.realm_hip_weights_release(handle))

    def weights_info(self, handle: int):
        t, n, k, nb = c_int(), c_size_t(), c_size_t(), c_size_t()
        self._check(self.lib.realm_hip_weights_info(handle, byref(t), byref(n), byref(k),
                                                    byref(nb)))
        return t.value, n.value, k.value, nb.value

    def weights_matmul(self, handle: int, x) -> np.ndarray:
        _, n, k, _ = self.weights_info(handle)
        x = np.ascontiguousarray(x, np.float32).reshape(-1, k)
        out = np.empty((x.shape[0], n), np.float32)
        self._check(self.lib.realm_hip_weights_matmul(handle, _ptr(x), x.shape[0], _ptr(out)))
        return out

    def lora_register(self, a, b, rank: int, alpha: float, in_dim: int, out_dim: int) -> int:
        a = np.ascontiguousarray(a)
        b = np.ascontiguousarray(b)
        if a.dtype == np.float16:
            dt = DTYPE_F16
            b = b.astype(np.float16)
        else:
            dt = DTYPE_F32
            a = a.astype(np.float32)
            b = b.astype(np.float32)
        h = c_uint64()
        self._check(self.lib.realm_hip_lora_register(dt, _ptr(a), _ptr(b), rank, alpha, in_dim,
                                                     out_dim, byref(h)))
        return h.value

    def lora_release(self, handle: int) -> None:
        self._check(self.lib.realm_hip_lora_release(handle))

    def lora_set_create(self, handles) -> int:
        arr = (c_uint64 * len(handles))(*handles)
        h = c_uint64()
        self._check(self.lib.realm_hip_lora_set_create(arr, len(handles), byref(h)))
        return h.value

    def lora_set_release(self, handle: int) -> None:
        self._check(self.lib.realm_hip_lora_set_release(handle))

    def multi_lora_matmul(self, weight_handle: int, set_handle: int, x, ids) -> np.ndarray:
        _, n, k, _ = self.weights_info(weight_handle)
        x = np.ascontiguousarray(x, np.float32).reshape(-1, k)
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty((x.shape[0], n), np.float32)
        self._check(self.lib.realm_hip_multi_lora_matmul(weight_handle, set_handle, _ptr(x),
                                                         x.shape[0], _ptr(ids), _ptr(out)))
        return out

    # --------------------------------------------------------- plumbing
    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def memcpy_dtod(self, dst: DeviceBuffer, src: DeviceBuffer, nbytes: int) -> None:
        if nbytes > min(dst.nbytes, src.nbytes):
            raise InvalidShape(f"copy of {nbytes} bytes exceeds a buffer")
        self._check(self.lib.realm_hip_memcpy_dtod(c_void_p(dst.ptr), c_void_p(src.ptr), nbytes))

    def stream(self) -> int:
        s = c_void_p()
        self._check(self.lib.realm_hip_stream(byref(s)))
        return s.value

    def synchronize(self) -> None:
        self._check(self.lib.realm_hip_device_synchronize())

    def event(self) -> int:
        e = c_void_p()
        self._check(self.lib.realm_hip_event_create(byref(e)))
        return e.value

    def record(self, event: int, stream: int | None = None) -> None:
        self._check(self.lib.realm_hip_event_record(c_void_p(event), c_void_p(stream or 0)))

    def elapsed_ms(self, start: int, stop: int) -> float:
        ms = c_float()
        self._check(self.lib.realm_hip_event_elapsed_ms(c_void_p(start), c_void_p(stop),
                                                        byref(ms)))
        return ms.value

    def matmul_dev(self, handle: int, d_x: int, batch: int, d_y: int, stream=None,
                   bf16: bool = False) -> None:
        fn = (self.lib.realm_hip_weights_matmul_bf16_dev if bf16
              else self.lib.realm_hip_weights_matmul_dev)
        self._check(fn(handle, c_void_p(d_x), batch, c_void_p(d_y), c_void_p(stream or 0)))

    def matmul_group_dev(self, handles, d_x: int, batch: int, d_ys, stream=None) -> None:
        hs = (c_uint64 * len(handles))(*handles)
        ys = (c_void_p * len(d_ys))(*d_ys)
        self._check(self.lib.realm_hip_weights_matmul_group_dev(
            hs, len(handles), c_void_p(d_x), batch, ys, c_void_p(stream or 0)))

    def graph_begin(self, stream: int) -> None:
        self._check(self.lib.realm_hip_graph_begin(c_void_p(stream)))

    def graph_end(self, stream: int) -> int:
        h = c_uint64()
        self._check(self.lib.realm_hip_graph_end(c_void_p(stream), byref(h)))
        return h.value

    def graph_launch(self, graph: int, stream: int | None = None) -> None:
        self._check(self.lib.realm_hip_graph_launch(graph, c_void_p(stream or 0)))

    def graph_release(self, graph: int) -> None:
        self._check(self.lib.realm_hip_graph_release(graph))

    def checksum(self, buf: "DeviceBuffer", nbytes: int | None = None) -> int:
        """XOR of the buffer's little-endian 32-bit words (tail zero-padded)."""
        out = ctypes.c_uint32()
        self._check(self.lib.realm_hip_checksum(c_void_p(buf.ptr),
                                                buf.nbytes if nbytes is None else nbytes,
                                                ctypes.byref(out)))
        return out.value

    def checksum_dev(self, d_buf: int, nbytes: int, d_partials: int, n_partials: int,
                     stream=None) -> None:
        self._check(self.lib.realm_hip_checksum_dev(c_void_p(d_buf), nbytes, c_void_p(d_partials),
                                                    n_partials, c_void_p(stream or 0)))

    def workspace_info(self, stream=None) -> tuple:
        """(bytes held, replaced buffers kept for live graphs, live graphs) of
        a stream's scratch buffers."""
        nb, ret, gr = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_int()
        self._check(self.lib.realm_hip_workspace_info(
            c_void_p(stream or 0), ctypes.byref(nb), ctypes.byref(ret), ctypes.byref(gr)))
        return nb.value, ret.value, gr.value

    def multi_lora_matmul_dev(self, wh: int, sh: int, d_x: int, batch: int, d_ids: int,
                              d_y: int, stream=None) -> None:
        self._check(self.lib.realm_hip_multi_lora_matmul_dev(
            wh, sh, c_void_p(d_x), batch, c_void_p(d_ids), c_void_p(d_y), c_void_p(stream or 0)))

    def multi_lora_matmul_group_dev(self, whs, shs, d_x: int, batch: int, d_ids: int, d_ys,
                                    stream=None) -> None:
        """Projections sharing x and the token adapter ids (e.g. q/k/v), each
        with its own adapter set: one activation prep, one base launch."""
        if len(whs) != len(shs) or len(whs) != len(d_ys):
            raise InvalidShape(INVALID_ARGUMENT, "one adapter set and output per weight")
        ws = (c_uint64 * len(whs))(*whs)
        ss = (c_uint64 * len(shs))(*shs)
        ys = (c_void_p * len(d_ys))(*d_ys)
        self._check(self.lib.realm_hip_multi_lora_matmul_group_dev(
            ws, ss, len(whs), c_void_p(d_x), batch, c_void_p(d_ids), ys, c_void_p(stream or 0)))

    # ------------------------------------------- element-wise layer ops
    def rms_norm_dev(self, d_x: int, d_weight: int, eps: float, rows: int, hidden: int,
                     d_out: int, d_residual: int = 0, d_sum: int = 0, stream=None) -> None:
        """RMSNorm per row (candle_neural_ops_backend.rs:32-60), optionally of
        x + residual (written to d_sum)."""
        self._check(self.lib.realm_hip_rms_norm_dev(
            c_void_p(d_x), c_void_p(d_residual or None), c_void_p(d_weight), eps, rows, hidden,
            c_void_p(d_sum or None), c_void_p(d_out), c_void_p(stream or 0)))

    def swiglu_dev(self, d_gate: int, d_up: int, n: int, d_out: int, stream=None) -> None:
        """silu(gate) * up (memory64_host.rs:2419-2425)."""
        self._check(self.lib.realm_hip_swiglu_dev(c_void_p(d_gate), c_void_p(d_up), n,
                                                  c_void_p(d_out), c_void_p(stream or 0)))

    def rope_dev(self, d_x: int, seq_len: int, num_heads: int, head_dim: int, start_pos: int,
                 theta: float, stream=None) -> None:
        """MultiHeadAttention::apply_rope in place (attention.rs:171-235)."""
        self._check(self.lib.realm_hip_rope_dev(c_void_p(d_x), seq_len, num_heads, head_dim,
                                                start_pos, theta, c_void_p(stream or 0)))

    def attention_dev(self, d_q: int, d_k_cache: int, d_v_cache: int, seq_len: int, kv_len: int,
                      position: int, num_heads: int, num_kv_heads: int, head_dim: int,
                      d_out: int, stream=None) -> None:
        """Causal GQA attention over a device KV cache (attention.rs:300-380)."""
        self._check(self.lib.realm_hip_attention_dev(
            c_void_p(d_q), c_void_p(d_k_cache), c_void_p(d_v_cache), seq_len, kv_len, position,
            num_heads, num_kv_heads, head_dim, c_void_p(d_out), c_void_p(stream or 0)))

    def kv_append_dev(self, d_k: int, d_v: int, seq_len: int, kv_dim: int, cur_len: int,
                      max_len: int, d_k_cache: int, d_v_cache: int, stream=None) -> None:
        """KVCache::append (kv_cache.rs:44-70) into device caches."""
        self._check(self.lib.realm_hip_kv_append_dev(
            c_void_p(d_k), c_void_p(d_v), seq_len, kv_dim, cur_len, max_len, c_void_p(d_k_cache),
            c_void_p(d_v_cache), c_void_p(stream or 0)))

    def add_dev(self, d_a: int, d_b: int, n: int, d_out: int, stream=None) -> None:
        self._check(self.lib.realm_hip_add_dev(c_void_p(d_a), c_void_p(d_b), n,
                                               c_void_p(d_out), c_void_p(stream or 0)))

    def forward_layer_dev(self, layer: "RealmLayer", d_hidden: int, seq_len: int, position: int,
                          d_k_cache: int, d_v_cache: int, max_seq_len: int, d_out: int,
                          stream=None) -> None:
        """realm_forward_layer on the device (memory64_host.rs:1915-2472)."""
        self._check(self.lib.realm_hip_forward_layer_dev(
            ctypes.byref(layer), c_void_p(d_hidden), seq_len, position, c_void_p(d_k_cache),
            c_void_p(d_v_cache), max_seq_len, c_void_p(d_out), c_void_p(stream or 0)))

    def forward_layers_dev(self, layers, d_hidden: int, seq_len: int, position: int,
                           d_k_caches, d_v_caches, max_seq_len: int, d_out: int,
                           stream=None) -> None:
        """Several device layers back to back, residual adds fused between them."""
        arr = (RealmLayer * len(layers))(*layers)
        kc = (c_void_p * len(layers))(*d_k_caches)
        vc = (c_void_p * len(layers))(*d_v_caches)
        self._check(self.lib.realm_hip_forward_layers_dev(
            arr, len(layers), c_void_p(d_hidden), seq_len, position, kc, vc, max_seq_len,
            c_void_p(d_out), c_void_p(stream or 0)))


class RealmLayer(ctypes.Structure):
    """struct realm_layer of include/realm_hip.h."""
    _fields_ = [("wq", c_uint64), ("wk", c_uint64), ("wv", c_uint64), ("wo", c_uint64),
                ("w_gate", c_uint64), ("w_up", c_uint64), ("w_down", c_uint64),
                ("attn_norm", c_void_p), ("ffn_norm", c_void_p),
                ("hidden", ctypes.c_uint32), ("num_heads", ctypes.c_uint32),
                ("num_kv_heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32),
                ("intermediate", ctypes.c_uint32), ("rms_norm_eps", ctypes.c_float),
                ("rope_theta", ctypes.c_float),
                # per-tenant LoRA: adapter sets per projection (0 = none), device
                # adapter slot per token
                ("lora_q", c_uint64), ("lora_k", c_uint64), ("lora_v", c_uint64),
                ("lora_o", c_uint64), ("lora_gate", c_uint64), ("lora_up", c_uint64),
                ("lora_down", c_uint64), ("d_adapter_ids", c_void_p)]


__all__ = ["HipGpuBackend", "RealmLayer", "RealmError", "InvalidShape", "BackendError",
           "DeviceBuffer", "DTYPE_F32", "DTYPE_F16"]

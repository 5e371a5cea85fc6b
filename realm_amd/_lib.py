"""ctypes binding of librealm_hip.so (the C ABI of include/realm_hip.h).

There is no fallback: if the library is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_size_t, c_uint16, c_uint32
from ctypes import c_uint64, c_uint8, c_void_p

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "librealm_hip.so")

# name -> (restype, argtypes), exactly the declarations of include/realm_hip.h
SIGNATURES = {
    "realm_hip_init": (c_int, [c_int]),
    "realm_hip_last_error": (c_char_p, []),
    "realm_hip_last_kernel": (c_char_p, []),
    "realm_hip_backend_name": (c_char_p, []),
    "realm_hip_set_nan_fallback": (c_int, [c_int]),
    "realm_hip_matmul": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t, c_uint32, c_uint32,
                                 c_uint32, c_void_p]),
    "realm_hip_matmul_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32,
                                     c_int, c_void_p]),
    "realm_hip_fused_dequant_matmul_q4k": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t,
                                                   c_size_t, c_size_t, c_size_t, c_void_p]),
    "realm_hip_fused_dequant_matmul_q6k": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t,
                                                   c_size_t, c_size_t, c_size_t, c_void_p]),
    "realm_hip_fused_dequant_matmul_q80": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t,
                                                   c_size_t, c_size_t, c_size_t, c_void_p]),
    "realm_hip_fused_dequant_matmul": (c_int, [c_int, c_void_p, c_size_t, c_void_p, c_size_t,
                                               c_size_t, c_size_t, c_size_t, c_void_p]),
    "realm_hip_candle_matmul": (c_int32, [c_void_p, c_size_t, c_uint32, c_uint32, c_uint32,
                                          c_uint32, c_uint32, c_uint32]),
    "realm_hip_candle_matmul_transposed": (c_int32, [c_void_p, c_size_t, c_uint32, c_uint32,
                                                     c_uint32, c_uint32, c_uint32, c_uint32]),
    "realm_hip_dequantize": (c_int, [c_int, c_void_p, c_size_t, c_size_t, c_void_p]),
    "realm_hip_weights_register": (c_int, [c_int, c_void_p, c_size_t, c_size_t, c_size_t,
                                           POINTER(c_uint64)]),
    "realm_hip_weights_release": (c_int, [c_uint64]),
    "realm_hip_weights_info": (c_int, [c_uint64, POINTER(c_int), POINTER(c_size_t),
                                       POINTER(c_size_t), POINTER(c_size_t)]),
    "realm_hip_weights_matmul": (c_int, [c_uint64, c_void_p, c_size_t, c_void_p]),
    "realm_hip_weights_matmul_dev": (c_int, [c_uint64, c_void_p, c_size_t, c_void_p, c_void_p]),
    "realm_hip_weights_matmul_noalloc_dev": (c_int, [c_uint64, c_void_p, c_size_t, c_void_p,
                                                     c_void_p]),
    "realm_hip_weights_matmul_group_dev": (c_int, [POINTER(c_uint64), c_size_t, c_void_p,
                                                   c_size_t, POINTER(c_void_p), c_void_p]),
    "realm_hip_weights_matmul_bf16_dev": (c_int, [c_uint64, c_void_p, c_size_t, c_void_p,
                                                  c_void_p]),
    "realm_hip_lora_register": (c_int, [c_int, c_void_p, c_void_p, c_size_t, c_float, c_size_t,
                                        c_size_t, POINTER(c_uint64)]),
    "realm_hip_lora_release": (c_int, [c_uint64]),
    "realm_hip_lora_set_create": (c_int, [POINTER(c_uint64), c_size_t, POINTER(c_uint64)]),
    "realm_hip_lora_set_release": (c_int, [c_uint64]),
    "realm_hip_multi_lora_matmul": (c_int, [c_uint64, c_uint64, c_void_p, c_size_t, c_void_p,
                                            c_void_p]),
    "realm_hip_multi_lora_matmul_dev": (c_int, [c_uint64, c_uint64, c_void_p, c_size_t,
                                                c_void_p, c_void_p, c_void_p]),
    "realm_hip_multi_lora_matmul_group_dev": (c_int, [POINTER(c_uint64), POINTER(c_uint64),
                                                      c_size_t, c_void_p, c_size_t, c_void_p,
                                                      POINTER(c_void_p), c_void_p]),
    "realm_hip_graph_begin": (c_int, [c_void_p]),
    "realm_hip_graph_end": (c_int, [c_void_p, POINTER(c_uint64)]),
    "realm_hip_graph_launch": (c_int, [c_uint64, c_void_p]),
    "realm_hip_graph_release": (c_int, [c_uint64]),
    "realm_hip_workspace_info": (c_int, [c_void_p, POINTER(c_size_t), POINTER(c_size_t),
                                         POINTER(c_int)]),
    "realm_hip_checksum_dev": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t, c_void_p]),
    "realm_hip_checksum": (c_int, [c_void_p, c_size_t, POINTER(c_uint32)]),
    "realm_hip_malloc": (c_int, [POINTER(c_void_p), c_size_t]),
    "realm_hip_free": (c_int, [c_void_p]),
    "realm_hip_memcpy_htod": (c_int, [c_void_p, c_void_p, c_size_t]),
    "realm_hip_memcpy_dtoh": (c_int, [c_void_p, c_void_p, c_size_t]),
    "realm_hip_memcpy_dtod": (c_int, [c_void_p, c_void_p, c_size_t]),
    "realm_hip_stream": (c_int, [POINTER(c_void_p)]),
    "realm_hip_stream_synchronize": (c_int, [c_void_p]),
    "realm_hip_device_synchronize": (c_int, []),
    "realm_hip_event_create": (c_int, [POINTER(c_void_p)]),
    "realm_hip_event_destroy": (c_int, [c_void_p]),
    "realm_hip_event_record": (c_int, [c_void_p, c_void_p]),
    "realm_hip_event_elapsed_ms": (c_int, [c_void_p, c_void_p, POINTER(c_float)]),
    "realm_hip_gguf_parse": (c_int, [c_void_p, c_size_t, POINTER(c_uint64)]),
    "realm_hip_gguf_info": (c_int, [c_uint64, POINTER(c_uint32), POINTER(c_uint64),
                                    POINTER(c_uint64), POINTER(c_uint64)]),
    "realm_hip_gguf_tensor": (c_int, [c_uint64, c_size_t, c_char_p, c_size_t, POINTER(c_int),
                                      POINTER(c_uint32), POINTER(c_uint64), POINTER(c_uint64),
                                      POINTER(c_uint64)]),
    "realm_hip_gguf_find": (c_int, [c_uint64, c_char_p, POINTER(c_size_t)]),
    "realm_hip_gguf_meta_u32": (c_int, [c_uint64, c_char_p, POINTER(c_uint32)]),
    "realm_hip_gguf_meta_str": (c_int, [c_uint64, c_char_p, c_char_p, c_size_t]),
    "realm_hip_gguf_config": (c_int, [c_uint64, c_void_p]),
    "realm_hip_gguf_register": (c_int, [c_uint64, c_void_p, c_size_t, POINTER(c_size_t)]),
    "realm_hip_gguf_weight": (c_int, [c_uint64, c_char_p, POINTER(c_uint64), POINTER(c_size_t),
                                      POINTER(c_size_t)]),
    "realm_hip_gguf_release": (c_int, [c_uint64]),
    "realm_hip_rms_norm_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_float, c_size_t, c_size_t,
                                       c_void_p, c_void_p, c_void_p]),
    "realm_hip_swiglu_dev": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p, c_void_p]),
    "realm_hip_rope_dev": (c_int, [c_void_p, c_size_t, c_size_t, c_size_t, c_size_t, c_float,
                                   c_void_p]),
    "realm_hip_attention_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_size_t,
                                        c_size_t, c_size_t, c_size_t, c_size_t, c_void_p,
                                        c_void_p]),
    "realm_hip_kv_append_dev": (c_int, [c_void_p, c_void_p, c_size_t, c_size_t, c_size_t,
                                        c_size_t, c_void_p, c_void_p, c_void_p]),
    "realm_hip_add_dev": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p, c_void_p]),
    "realm_hip_forward_layer_dev": (c_int, [c_void_p, c_void_p, c_size_t, c_size_t, c_void_p,
                                            c_void_p, c_size_t, c_void_p, c_void_p]),
    "realm_hip_forward_layers_dev": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t, c_size_t,
                                             c_void_p, c_void_p, c_size_t, c_void_p, c_void_p]),
    "realm_hip_fused_dequant_matmul_q40": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t,
                                                   c_size_t, c_size_t, c_size_t, c_void_p]),
    "realm_hip_fused_dequant_matmul_q41": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t,
                                                   c_size_t, c_size_t, c_size_t, c_void_p]),
    "realm_hip_fused_dequant_matmul_q50": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t,
                                                   c_size_t, c_size_t, c_size_t, c_void_p]),
    "realm_hip_fused_dequant_matmul_q51": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t,
                                                   c_size_t, c_size_t, c_size_t, c_void_p]),
    "realm_hip_fused_dequant_matmul_q81": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t,
                                                   c_size_t, c_size_t, c_size_t, c_void_p]),
    "realm_hip_fused_dequant_matmul_q5k": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t,
                                                   c_size_t, c_size_t, c_size_t, c_void_p]),
    "realm_hip_fused_dequant_matmul_q8k": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t,
                                                   c_size_t, c_size_t, c_size_t, c_void_p]),
    "realm_hip_fused_dequant_matmul_q2k": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t,
                                                   c_size_t, c_size_t, c_size_t, c_void_p]),
    "realm_hip_fused_dequant_matmul_q3k": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t,
                                                   c_size_t, c_size_t, c_size_t, c_void_p]),
}

_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the library and bind every declared symbol (raises if absent)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run `python -m realm_amd.build`")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


__all__ = ["load", "LIB_PATH", "SIGNATURES", "c_uint8", "c_uint16"]

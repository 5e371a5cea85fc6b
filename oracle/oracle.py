"""ctypes wrapper of oracle/build/librealm_oracle.so -- TEST INFRASTRUCTURE ONLY.

The checker the HIP path is compared against; see realm_oracle.c for the
reference citation of every function.  Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg may use it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, c_double, c_float, c_int, c_int32, c_size_t, c_uint8, c_uint16
from ctypes import c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "librealm_oracle.so")

GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 8, 12, 14
GGML_Q4_0, GGML_Q4_1, GGML_Q5_0, GGML_Q5_1, GGML_Q8_1 = 2, 3, 6, 7, 9
GGML_Q2_K, GGML_Q3_K, GGML_Q5_K, GGML_Q8_K = 10, 11, 13, 15
# bytes per block and elements per block of every format restated here (the
# reference's own #[repr(C)] sizes for Q2_K/Q3_K/Q5_K/Q8_K)
BLOCK_BYTES = {GGML_Q4_K: 144, GGML_Q6_K: 210, GGML_Q8_0: 34, GGML_Q4_0: 18, GGML_Q4_1: 20,
               GGML_Q5_0: 22, GGML_Q5_1: 24, GGML_Q8_1: 36, GGML_Q2_K: 116, GGML_Q3_K: 196,
               GGML_Q5_K: 178, GGML_Q8_K: 292}
BLOCK_ELEMS = {t: (256 if t in (GGML_Q4_K, GGML_Q6_K, GGML_Q2_K, GGML_Q3_K, GGML_Q5_K,
                                GGML_Q8_K) else 32) for t in BLOCK_BYTES}
OK, INVALID_ARGUMENT, MODEL_PARSE_ERROR, PANIC = 0, 3, 4, -1

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        vp, sz, fp = c_void_p, c_size_t, c_float
        sig = {
            "ro_f16_to_f32": (c_float, [c_uint16]),
            "ro_f32_to_f16": (c_uint16, [c_float]),
            "ro_get_scale_min_k4": (None, [c_int, vp, POINTER(c_uint8), POINTER(c_uint8)]),
            "ro_dequantize_q4_k": (c_int, [vp, vp]),
            "ro_dequantize_q6_k": (c_int, [vp, vp]),
            "ro_dequantize_q8_0": (c_int, [vp, vp]),
            "ro_dequantize_tensor": (c_int, [vp, sz, c_int, sz, vp]),
            "ro_fused_q4k": (c_int, [vp, sz, vp, sz, vp, sz, sz, sz, c_int]),
            "ro_fused_q6k": (c_int, [vp, sz, vp, sz, vp, sz, sz, sz, c_int]),
            "ro_fused_q80": (c_int, [vp, sz, vp, sz, vp, sz, sz, sz]),
            "ro_candle_fused": (c_int, [c_int, vp, sz, vp, sz, vp, sz, sz, sz]),
            "ro_matmul_f32": (c_int, [vp, sz, vp, sz, vp, sz, sz, sz]),
            "ro_matmul_transposed": (c_int, [vp, sz, vp, sz, vp, sz, sz, sz]),
            "ro_lora_apply_to_weights": (c_int, [vp, sz, vp, sz, vp, sz, sz, fp, sz, sz, vp]),
            "ro_multi_lora_delta": (c_int, [vp, sz, sz, sz, vp, sz, vp, vp, vp, vp, vp]),
            "ro_matvec_f64": (None, [vp, vp, vp, sz, sz, sz]),
            "ro_fused_parallel": (c_int, [c_int, vp, vp, vp, sz, sz, sz, c_int]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return c_void_p(0 if a is None else a.ctypes.data)


def f16_to_f32(h: int) -> float:
    return lib().ro_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().ro_f32_to_f16(f)


def get_scale_min_k4(j: int, scales) -> tuple[int, int]:
    s = np.ascontiguousarray(scales, np.uint8)
    sc, m = c_uint8(), c_uint8()
    lib().ro_get_scale_min_k4(j, _p(s), ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


def dequantize_tensor(ggml_type: int, data, element_count: int):
    """(status, f32 array) with quant.rs dequantize_tensor semantics."""
    raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
    out = np.zeros(max(element_count, 1), np.float32)
    rc = lib().ro_dequantize_tensor(_p(raw), raw.size, ggml_type, element_count, _p(out))
    return rc, out[:element_count]


def dequantize(ggml_type: int, blocks) -> np.ndarray:
    raw = np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
    per, bb = BLOCK_ELEMS[ggml_type], BLOCK_BYTES[ggml_type]
    rc, out = dequantize_tensor(ggml_type, raw, (raw.size // bb) * per)
    assert rc == OK, rc
    return out


def fused(ggml_type: int, blocks, x, batch: int, n: int, k: int, nan_fallback: bool = True):
    """fused.rs semantics; returns (status, out)."""
    raw = np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
    bb = {GGML_Q4_K: 144, GGML_Q6_K: 210, GGML_Q8_0: 34}[ggml_type]
    nb = raw.size // bb
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(max(batch * n, 1), np.float32)
    L = lib()
    if ggml_type == GGML_Q4_K:
        rc = L.ro_fused_q4k(_p(raw), nb, _p(x), x.size, _p(out), batch, n, k, int(nan_fallback))
    elif ggml_type == GGML_Q6_K:
        rc = L.ro_fused_q6k(_p(raw), nb, _p(x), x.size, _p(out), batch, n, k, int(nan_fallback))
    else:
        rc = L.ro_fused_q80(_p(raw), nb, _p(x), x.size, _p(out), batch, n, k)
    return rc, out[:batch * n]


def candle_fused(ggml_type: int, blocks, x, batch: int, n: int, k: int):
    """CandleCpuBackend semantics; returns (status, out)."""
    raw = np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
    bb = BLOCK_BYTES[ggml_type]
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(max(batch * n, 1), np.float32)
    rc = lib().ro_candle_fused(ggml_type, _p(raw), raw.size // bb, _p(x), x.size, _p(out),
                               batch, n, k)
    return rc, out[:batch * n]


def matmul_f32(a, b, m: int, k: int, n: int):
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    b = np.ascontiguousarray(b, np.float32).reshape(-1)
    c = np.zeros(max(m * n, 1), np.float32)
    rc = lib().ro_matmul_f32(_p(a), a.size, _p(b), b.size, _p(c), m, k, n)
    return rc, c[:m * n]


def matmul_transposed(a, bt, m: int, k: int, n: int):
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    bt = np.ascontiguousarray(bt, np.float32).reshape(-1)
    c = np.zeros(max(m * n, 1), np.float32)
    rc = lib().ro_matmul_transposed(_p(a), a.size, _p(bt), bt.size, _p(c), m, k, n)
    return rc, c[:m * n]


def lora_apply_to_weights(base, lora_a, lora_b, rank: int, alpha: float, out_dim: int,
                          in_dim: int):
    base = np.ascontiguousarray(base, np.float32).reshape(-1)
    a = np.ascontiguousarray(lora_a, np.float32).reshape(-1)
    b = np.ascontiguousarray(lora_b, np.float32).reshape(-1)
    out = np.empty_like(base)
    rc = lib().ro_lora_apply_to_weights(_p(base), base.size, _p(a), a.size, _p(b), b.size,
                                        rank, alpha, out_dim, in_dim, _p(out))
    return rc, out


def multi_lora_delta(x, ids, adapters, y):
    """Adds the unmerged LoRA delta to y in place.  adapters: list of
    (A [r,k] f32, B [n,r] f32, rank, alpha)."""
    x = np.ascontiguousarray(x, np.float32)
    batch, k = x.shape
    n = y.shape[1]
    ids = np.ascontiguousarray(ids, np.int32)
    As = [np.ascontiguousarray(a, np.float32) for a, _, _, _ in adapters]
    Bs = [np.ascontiguousarray(b, np.float32) for _, b, _, _ in adapters]
    ap = (c_void_p * len(adapters))(*[a.ctypes.data for a in As])
    bp = (c_void_p * len(adapters))(*[b.ctypes.data for b in Bs])
    ranks = np.array([r for _, _, r, _ in adapters], np.int32)
    alphas = np.array([al for _, _, _, al in adapters], np.float32)
    assert y.dtype == np.float32 and y.flags.c_contiguous
    rc = lib().ro_multi_lora_delta(_p(x), batch, k, n, _p(ids), len(adapters), ap, bp,
                                   _p(ranks), _p(alphas), _p(y))
    assert rc == OK, rc
    return y


def matvec_f64(w, x, batch: int, n: int, k: int) -> np.ndarray:
    w = np.ascontiguousarray(w, np.float32).reshape(-1)
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    y = np.zeros(batch * n, np.float64)
    lib().ro_matvec_f64(_p(w), _p(x), _p(y), batch, n, k)
    return y


def fused_parallel(ggml_type: int, blocks, x, batch: int, n: int, k: int, threads: int = 0):
    """Row-parallel CPU timing variant; returns (threads_used, out)."""
    raw = np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(batch * n, np.float32)
    used = lib().ro_fused_parallel(ggml_type, _p(raw), _p(x), _p(out), batch, n, k, threads)
    return used, out


_ = (c_double, c_int32)

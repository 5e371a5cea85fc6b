"""The C-ABI library loads and exports exactly what include/realm_hip.h
declares, and the ctypes binding matches the header.  No GPU calls."""
import ctypes
import os
import re
import subprocess

import pytest

from conftest import REPO

HEADER = os.path.join(REPO, "include", "realm_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(realm_hip_\w+)\s*\(", text))


def test_header_declares_the_boundary():
    names = declared_functions()
    for n in ("realm_hip_init", "realm_hip_last_error", "realm_hip_backend_name",
              "realm_hip_matmul", "realm_hip_fused_dequant_matmul_q4k",
              "realm_hip_fused_dequant_matmul_q6k", "realm_hip_fused_dequant_matmul_q80",
              "realm_hip_candle_matmul", "realm_hip_candle_matmul_transposed",
              "realm_hip_dequantize", "realm_hip_weights_register",
              "realm_hip_multi_lora_matmul", "realm_hip_lora_register"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from realm_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in sorted(declared_functions()):
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (realm_hip_\w+)", out))
    assert exported == declared_functions()


def test_ctypes_binding_matches_header():
    from realm_amd import _lib
    assert set(_lib.SIGNATURES) == declared_functions()


def test_code_object_is_embedded_for_gfx950():
    from realm_amd import _lib, build
    paths = [os.path.join(build.LIB_DIR, name + ".hsaco") for name, _, _ in build.HSACO_UNITS]
    if not all(os.path.exists(p) for p in paths):
        pytest.skip("code objects not built")
    lib = open(_lib.LIB_PATH, "rb").read()
    blobs = b""
    for p in paths:
        blob = open(p, "rb").read()
        assert blob[:4] == b"\x7fELF" and b"gfx950" in blob
        assert blob[:4096] in lib  # embedded verbatim
        blobs += blob
    for k in (b"realm_gemv_q4k_l64_u1_d2_m1", b"realm_gemv_q6k_l64_u3_d2_m4",
              b"realm_gemv_q80_l32_u1_d1_m1", b"realm_gemm_q4k_p4_bf16", b"realm_dequant_q6k",
              b"realm_lora_shrink_q4k_f32", b"realm_lora_shrink_q6k_f32_o1", b"realm_dense_f32",
              b"realm_gemm_q4k_t4112b2", b"realm_gemm_q6kw_t4112p2", b"realm_xprep_q4k_o1",
              b"realm_gemm_tiled_reduce", b"realm_gemm_tiled_reduce_lora",
              b"realm_xprep_lora_q4k_o1", b"realm_xprep_lora_q6k",
              b"realm_gemv_q8m_l64_u1_d1_m1", b"realm_gemv_q8m_l32_u1_d2_m4_t4",
              b"realm_repack_q32", b"realm_dequant_q8m", b"realm_gemm_q80_t4112b2",
              b"realm_gemm_q80_t4111p2", b"realm_xprep_lora_q80_o1", b"realm_dense_f32_m32",
              b"realm_dense_f32_m64", b"realm_gemv_q4k_l64_u1_d1_m4_n",
              b"realm_gemv_q6k_l64_u3_d2_m1_s", b"realm_gemv_q80_l16_u1_d3_m4_n",
              b"realm_attention_tiled_h32", b"realm_attention_tiled_h256",
              b"realm_xprep_q4k_o1_t256", b"realm_xprep_q80_t256", b"realm_xprep_q6k_o1_t512",
              b"realm_rope_qk_tab", b"realm_rope_table_seq"):
        assert k in blobs

"""GGUF block layouts of the quantized path as numpy structured dtypes.

Byte-identical to the #[repr(C)] block structs of the reference
(crates/realm-core/src/quant.rs: BlockQ8_0 :52-59, BlockQ4_K :97-107,
BlockQ6_K :191-198) and to the ggml tensor type ids of
crates/realm-core/src/formats/gguf.rs:458-480.
"""
import numpy as np

GGML_Q8_0 = 8
GGML_Q4_K = 12
GGML_Q6_K = 14

QK_K = 256
QK8_0 = 32

Q4K_DTYPE = np.dtype([("d", "<u2"), ("dmin", "<u2"), ("scales", "u1", (12,)),
                      ("qs", "u1", (128,))])
Q6K_DTYPE = np.dtype([("ql", "u1", (128,)), ("qh", "u1", (64,)), ("scales", "i1", (16,)),
                      ("d", "<u2")])
Q80_DTYPE = np.dtype([("scale", "<u2"), ("quants", "i1", (32,))])

assert Q4K_DTYPE.itemsize == 144 and Q6K_DTYPE.itemsize == 210 and Q80_DTYPE.itemsize == 34

DTYPES = {GGML_Q4_K: Q4K_DTYPE, GGML_Q6_K: Q6K_DTYPE, GGML_Q8_0: Q80_DTYPE}
BLOCK_ELEMS = {GGML_Q4_K: QK_K, GGML_Q6_K: QK_K, GGML_Q8_0: QK8_0}
NAMES = {GGML_Q4_K: "Q4_K", GGML_Q6_K: "Q6_K", GGML_Q8_0: "Q8_0"}


def n_blocks(ggml_type: int, n: int, k: int) -> int:
    return n * (k // BLOCK_ELEMS[ggml_type])


def weight_bytes(ggml_type: int, n: int, k: int) -> int:
    return n_blocks(ggml_type, n, k) * DTYPES[ggml_type].itemsize

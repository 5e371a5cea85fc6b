"""Seeded synthetic inputs for the benchmark configurations.

Every tensor comes from numpy's PCG64 generator (``numpy.random.default_rng``)
seeded once per workload, drawn in a fixed order.  Distributions follow the
workload definitions:

* Q4_K block: d, dmin = f16(|N(0,1)| * 1e-3); 12 scale bytes uniform (that is,
  8 six-bit scales and 8 six-bit mins uniform in 0..63); 128 qs bytes uniform
  (4-bit quants uniform in 0..15).
* Q6_K block: ql, qh bytes uniform (6-bit quants uniform in 0..63); sub-scales
  int8 uniform in -32..31; d as above.
* Q8_0 block: d as above; 32 int8 quants uniform in -127..127.
* activations: f32 N(0,1) (decode) or bf16-rounded N(0,1) (prefill).
* LoRA: A [r, in] f16 N(0, 1/sqrt(in)), B [out, r] f16 N(0, 0.01), alpha = 16,
  ranks drawn from {8, 16, 64}; token adapter ids Zipf(1.1) over the tenants,
  replaced by -1 (no adapter) with probability 0.1.
"""
from __future__ import annotations

import numpy as np

from .formats import GGML_Q4_K, GGML_Q6_K, GGML_Q8_0, Q4K_DTYPE, Q6K_DTYPE, Q80_DTYPE


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def _f16_scale(g: np.random.Generator, count: int) -> np.ndarray:
    return (np.abs(g.standard_normal(count)) * 1e-3).astype(np.float16).view(np.uint16)


def q4k_blocks(g: np.random.Generator, n: int, k: int) -> np.ndarray:
    nb = n * (k // 256)
    b = np.empty(nb, Q4K_DTYPE)
    b["d"] = _f16_scale(g, nb)
    b["dmin"] = _f16_scale(g, nb)
    b["scales"] = g.integers(0, 256, (nb, 12), dtype=np.uint8)
    b["qs"] = g.integers(0, 256, (nb, 128), dtype=np.uint8)
    return b


def q6k_blocks(g: np.random.Generator, n: int, k: int) -> np.ndarray:
    nb = n * (k // 256)
    b = np.empty(nb, Q6K_DTYPE)
    b["ql"] = g.integers(0, 256, (nb, 128), dtype=np.uint8)
    b["qh"] = g.integers(0, 256, (nb, 64), dtype=np.uint8)
    b["scales"] = g.integers(-32, 32, (nb, 16), dtype=np.int8)
    b["d"] = _f16_scale(g, nb)
    return b


def q80_blocks(g: np.random.Generator, n: int, k: int) -> np.ndarray:
    nb = n * (k // 32)
    b = np.empty(nb, Q80_DTYPE)
    b["scale"] = _f16_scale(g, nb)
    b["quants"] = g.integers(-127, 128, (nb, 32), dtype=np.int8)
    return b


def blocks(g: np.random.Generator, ggml_type: int, n: int, k: int) -> np.ndarray:
    if ggml_type == GGML_Q4_K:
        return q4k_blocks(g, n, k)
    if ggml_type == GGML_Q6_K:
        return q6k_blocks(g, n, k)
    if ggml_type == GGML_Q8_0:
        return q80_blocks(g, n, k)
    raise ValueError(f"unsupported ggml type {ggml_type}")


def activations(g: np.random.Generator, m: int, k: int) -> np.ndarray:
    return g.standard_normal((m, k), dtype=np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16, returned as uint16 bits."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def activations_bf16(g: np.random.Generator, m: int, k: int) -> np.ndarray:
    """bf16 activations as uint16 bits."""
    return f32_to_bf16_bits(g.standard_normal((m, k), dtype=np.float32))


def lora_adapter(g: np.random.Generator, rank: int, in_dim: int, out_dim: int):
    """(A [rank, in] f16, B [out, rank] f16)."""
    a = (g.standard_normal((rank, in_dim)) / np.sqrt(in_dim)).astype(np.float16)
    b = (g.standard_normal((out_dim, rank)) * 0.01).astype(np.float16)
    return a, b


def adapter_ids(g: np.random.Generator, m: int, n_adapters: int, s: float = 1.1,
                p_none: float = 0.1) -> np.ndarray:
    w = 1.0 / np.arange(1, n_adapters + 1) ** s
    ids = g.choice(n_adapters, size=m, p=w / w.sum()).astype(np.int32)
    ids[g.random(m) < p_none] = -1
    return ids

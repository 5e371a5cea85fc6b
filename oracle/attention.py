"""Attention of realm_forward_layer restated in numpy -- TEST INFRASTRUCTURE ONLY.

  rope       MultiHeadAttention::apply_rope (crates/realm-models/src/
             attention.rs:171-235): interleaved pairs, freq =
             1 / theta^(i / head_dim) in f32, angle = pos * freq, then
             (x0 cos - x1 sin, x0 sin + x1 cos).
  kv_append  KVCache::append (crates/realm-models/src/kv_cache.rs:44-70),
             overflow -> error.
  attention  MultiHeadAttention::compute_attention (attention.rs:300-380)
             with StandardAttention (crates/realm-runtime/src/attention/
             standard.rs:36-210): repeat_kv for GQA, causal mask
             j > position + i -> -inf, scores (q . k) * 1/sqrt(head_dim),
             softmax with the max subtracted and division by the sum,
             output sum_j p_j v_j; all in f32.
"""
from __future__ import annotations

import numpy as np


def rope(x, start_pos: int, seq_len: int, num_heads: int, head_dim: int, theta: float):
    x = np.array(x, np.float32).reshape(seq_len, num_heads, head_dim)
    i = np.arange(0, head_dim, 2, dtype=np.float32)
    freq = (np.float32(1.0) / np.power(np.float32(theta), i / np.float32(head_dim))).astype(
        np.float32)
    for s in range(seq_len):
        ang = (np.float32(start_pos + s) * freq).astype(np.float32)
        c, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
        x0, x1 = x[s, :, 0::2].copy(), x[s, :, 1::2].copy()
        x[s, :, 0::2] = x0 * c - x1 * sn
        x[s, :, 1::2] = x0 * sn + x1 * c
    return x.reshape(-1)


class KVCacheError(Exception):
    pass


def kv_append(k_cache, v_cache, cur_len: int, max_len: int, k, v, kv_dim: int) -> int:
    n = len(k) // kv_dim
    if cur_len + n > max_len:
        raise KVCacheError(f"KV cache overflow: {cur_len} + {n} > {max_len}")
    k_cache[cur_len * kv_dim:(cur_len + n) * kv_dim] = k
    v_cache[cur_len * kv_dim:(cur_len + n) * kv_dim] = v
    return cur_len + n


def attention(q, k, v, seq_len: int, kv_len: int, position: int, num_heads: int,
              num_kv_heads: int, head_dim: int):
    q = np.asarray(q, np.float32).reshape(seq_len, num_heads, head_dim)
    k = np.asarray(k, np.float32).reshape(kv_len, num_kv_heads, head_dim)
    v = np.asarray(v, np.float32).reshape(kv_len, num_kv_heads, head_dim)
    n_rep = num_heads // num_kv_heads
    kr = np.repeat(k, n_rep, axis=1)   # head h <- kv head h // n_rep
    vr = np.repeat(v, n_rep, axis=1)
    scale = np.float32(1.0 / np.sqrt(np.float32(head_dim)))
    out = np.zeros((seq_len, num_heads, head_dim), np.float32)
    for h in range(num_heads):
        scores = (q[:, h, :] @ kr[:, h, :].T).astype(np.float32) * scale
        for i in range(seq_len):
            row = scores[i].copy()
            row[np.arange(kv_len) > position + i] = -np.inf
            # the max is a fold of f32::max from -inf: NaN scores are skipped
            # (standard.rs:114-116)
            kept = row[~np.isnan(row)]
            mx = np.max(kept) if kept.size else -np.inf
            e = np.where(np.isfinite(row), np.exp(row - mx), 0).astype(np.float32)
            s = np.float32(e.sum(dtype=np.float32))
            if s > 0:
                e = (e / s).astype(np.float32)
            out[i, h, :] = (e @ vr[:, h, :]).astype(np.float32)
    return out.reshape(-1)


def forward_layer(matmul, x, w, norms, cfg, k_cache, v_cache, position: int, seq_len: int):
    """realm_forward_layer's decoder layer (crates/realm-runtime/src/
    memory64_host.rs:2059-2458) composed from the restated steps:
    matmul(name, x, m) -> [m, n] is the caller's fused dequant x matmul
    (the oracle's candle_fused); w names the seven projections; norms holds
    the two norm vectors; the caches are [max_len * kv_dim] arrays whose
    rows position.. are written (KVCache::append).  Returns [seq_len, hidden]."""
    from oracle import layer_ops as lo
    H, heads, kvh, hd = cfg["hidden"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
    kv_dim = kvh * hd
    eps, theta = cfg["eps"], cfg["theta"]
    x = np.asarray(x, np.float32).reshape(seq_len, H)
    normed, _ = lo.rms_norm(x, norms["attn"], eps)
    q = matmul("wq", normed, seq_len).reshape(-1)
    k = matmul("wk", normed, seq_len).reshape(-1)
    v = matmul("wv", normed, seq_len).reshape(-1)
    q = rope(q, position, seq_len, heads, hd, theta)
    k = rope(k, position, seq_len, kvh, hd, theta)
    kv_len = kv_append(k_cache, v_cache, position, len(k_cache) // kv_dim, k, v, kv_dim)
    att = attention(q, k_cache[:kv_len * kv_dim], v_cache[:kv_len * kv_dim], seq_len, kv_len,
                    position, heads, kvh, hd)
    o = matmul("wo", att.reshape(seq_len, H), seq_len)
    ffn_normed, h2 = lo.rms_norm(x, norms["ffn"], eps, residual=o)
    gate = matmul("w_gate", ffn_normed, seq_len)
    up = matmul("w_up", ffn_normed, seq_len)
    act = lo.swiglu(gate, up)
    down = matmul("w_down", act, seq_len)
    return (h2 + down).astype(np.float32)

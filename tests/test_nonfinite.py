"""Activations the fast paths cannot scale: NaN, +Inf, -Inf, all-subnormal,
tiny (max |x| below 2^-60) and huge (above 2^100) tokens, on every product
path (one- and multi-token GEMV, grouped GEMV, small-batch MFMA tiles, the
LDS-tiled kernel with and without a K split, bf16 prefill, Q8_0), and
non-finite attention scores.

The reference computes such products in f32 (candle_cpu_backend.rs:92-114,
fused.rs:229-374): NaN in x gives NaN, an Inf gives +-Inf by the sign of the
weights it meets and NaN where it meets a zero weight or both signs.  The
GPU must put NaN and +-Inf exactly where the oracle does and agree within
1e-3 relative L2 on the finite entries of every token.  The reference's
softmax gives a non-finite score weight 0 and takes its max with f32::max
(NaN skipped; crates/realm-runtime/src/attention/standard.rs:114-126).
"""
import zlib

import numpy as np
import pytest

from oracle import attention as oa
from realm_amd import synth
from realm_amd.formats import GGML_Q4_K, GGML_Q6_K, GGML_Q8_0, NAMES

from conftest import rel_l2

REL_TOL = 1e-3


def special_tokens(g, m, k, bf16=False):
    """m tokens: a normal one, then one each of NaN, +Inf, -Inf, +Inf and
    -Inf together, all-subnormal, tiny, huge, then normal ones."""
    x = g.standard_normal((m, k)).astype(np.float32)
    kinds = ["normal", "nan", "+inf", "-inf", "both", "subnormal", "tiny", "huge"]
    for i, kind in enumerate(kinds[:m]):
        p = g.integers(0, k, 3)
        if kind == "nan":
            x[i, p[0]] = np.nan
        elif kind == "+inf":
            x[i, p[0]] = np.inf
        elif kind == "-inf":
            x[i, p[1]] = -np.inf
        elif kind == "both":
            x[i, p[0]], x[i, p[2]] = np.inf, -np.inf
        elif kind == "subnormal":
            x[i] *= np.float32(1e-39)
        elif kind == "tiny":
            x[i] *= np.float32(1e-25)
        elif kind == "huge":
            x[i] *= np.float32(1e33)
    if bf16:
        xb = synth.f32_to_bf16_bits(x)
        return xb, synth.bf16_bits_to_f32(xb)
    return x, x


def assert_same_class(got, ref, tag):
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32).reshape(got.shape)
    assert np.array_equal(np.isnan(got), np.isnan(ref)), f"{tag}: NaN positions"
    assert np.array_equal(np.isposinf(got), np.isposinf(ref)), f"{tag}: +Inf positions"
    assert np.array_equal(np.isneginf(got), np.isneginf(ref)), f"{tag}: -Inf positions"
    for i in range(got.shape[0]):
        fin = np.isfinite(ref[i])
        if fin.any():
            err = rel_l2(got[i][fin], ref[i][fin])
            assert err < REL_TOL, f"{tag}: token {i} finite rel_l2 {err:.3e}"


# ----------------------------------------------------------------- CPU

def test_oracle_softmax_nonfinite_scores():
    """The oracle's attention follows standard.rs on non-finite scores: a
    NaN score is skipped by the max and weighted 0; an +Inf score makes the
    max +Inf, so every weight is 0 and the output is 0; -Inf (a masked key)
    is weighted 0."""
    hd, heads = 4, 1
    q = np.ones(hd, np.float32)
    v = np.arange(3 * hd, dtype=np.float32)
    k = np.ones(3 * hd, np.float32)
    k[:hd] = np.nan  # key 0: NaN score
    out = oa.attention(q, k, v, 1, 3, 2, heads, 1, hd)
    assert np.allclose(out, v.reshape(3, hd)[1:].mean(0))  # keys 1, 2 equal
    k2 = np.ones(3 * hd, np.float32)
    k2[hd] = np.inf  # key 1: +Inf score
    assert np.array_equal(oa.attention(q, k2, v, 1, 3, 2, heads, 1, hd), np.zeros(hd, np.float32))
    k3 = np.ones(3 * hd, np.float32)
    k3[2 * hd] = -np.inf  # key 2: -Inf score
    assert np.allclose(oa.attention(q, k3, v, 1, 3, 2, heads, 1, hd), v.reshape(3, hd)[:2].mean(0))


def test_oracle_nonfinite_products(oracle):
    """The oracle's f32 product (the GPU's reference) on special tokens:
    NaN rows, +-Inf by weight sign, finite tokens finite."""
    g = synth.rng(8000)
    n, k = 64, 512
    blocks = synth.blocks(g, GGML_Q4_K, n, k)
    x, _ = special_tokens(g, 8, k)
    rc, y = oracle.candle_fused(GGML_Q4_K, blocks, x, 8, n, k)
    y = y.reshape(8, n)
    assert rc == 0
    assert np.isnan(y[1]).all()
    w = oracle.dequantize(GGML_Q4_K, blocks).reshape(n, k)
    p = int(np.flatnonzero(np.isposinf(x[2]))[0])
    want = np.where(w[:, p] > 0, np.inf, np.where(w[:, p] < 0, -np.inf, np.nan))
    assert np.array_equal(np.isposinf(y[2]), np.isposinf(want))
    assert np.array_equal(np.isnan(y[2]), np.isnan(want))
    for i in (0, 5, 6, 7):
        assert np.isfinite(y[i]).all()


# ----------------------------------------------------------------- GPU

def _run(backend, t, blocks, n, k, x, bf16=False, group=1):
    m = x.shape[0]
    hs = [backend.register_weights(t, blocks, n, k) for _ in range(group)]
    dx = backend.alloc(x.nbytes).upload(x)
    dys = [backend.alloc(m * n * 4) for _ in range(group)]
    try:
        if group == 1:
            backend.matmul_dev(hs[0], dx.ptr, m, dys[0].ptr, bf16=bf16)
        else:
            backend.matmul_group_dev(hs, dx.ptr, m, [d.ptr for d in dys])
        backend.synchronize()
        kernel = backend.last_kernel()
        outs = [d.download(np.float32, m * n).reshape(m, n) for d in dys]
    finally:
        for h in hs:
            backend.release_weights(h)
        for d in [dx] + dys:
            d.close()
    return outs, kernel


CASES = [  # (format, m, k, group, bf16, forced tile, forced K split, kernel prefix)
    (GGML_Q4_K, 1, 4096, 1, False, None, None, "realm_gemv_q4k_l64_u1"),
    (GGML_Q4_K, 1, 4096, 3, False, None, None, "realm_gemv_q4k_l64_u1"),
    (GGML_Q4_K, 1, 11008, 1, False, None, None, "realm_gemv_q4k_l64_u3"),
    (GGML_Q6_K, 1, 11008, 1, False, None, None, "realm_gemv_q6k_l64_u3"),
    (GGML_Q8_0, 1, 4096, 1, False, None, None, "realm_gemv_q80"),
    (GGML_Q4_K, 2, 4096, 1, False, None, None, "realm_gemv_q4k"),
    (GGML_Q6_K, 4, 4096, 2, False, None, None, "realm_gemv_q6k"),
    (GGML_Q4_K, 6, 2048, 1, False, None, None, "realm_gemm_q4k_s1"),
    (GGML_Q4_K, 37, 2048, 1, False, "t4112p2", "1", "realm_gemm_q4k_t4112p2"),
    (GGML_Q6_K, 37, 2048, 2, False, "t4112p2", "4", "realm_gemm_tiled_reduce"),
    (GGML_Q6_K, 70, 2048, 1, False, "t4112s2", "1", "realm_gemm_q6k_t4112s2"),
    (GGML_Q4_K, 64, 2048, 1, True, "t4112b2", "1", "realm_gemm_q4k_t4112b2"),
    (GGML_Q8_0, 37, 2048, 1, False, None, None, "realm_gemm_tiled_reduce"),
    (GGML_Q8_0, 37, 2048, 1, False, "t4112p2", "1", "realm_gemm_q80_t4112p2"),
    (GGML_Q8_0, 64, 2048, 1, True, "t4112b2", "1", "realm_gemm_q80_t4112b2"),
    (GGML_Q8_0, 37, 2112, 1, False, None, None, "realm_gemm_q80_d4"),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=[f"{NAMES[c[0]]}-m{c[1]}-k{c[2]}-g{c[3]}"
                                             f"{'-bf16' if c[4] else ''}-{c[5] or ''}{c[6] or ''}"
                                             for c in CASES])
def test_nonfinite_activations(backend, oracle, monkeypatch, case):
    t, m, k, group, bf16, tile, ks, prefix = case
    if tile:
        monkeypatch.setenv("REALM_GEMM_TILE", tile)
        monkeypatch.setenv("REALM_GEMM_KS", ks)
    g = synth.rng(zlib.crc32(repr(case).encode()) % 100000)
    n = 200
    blocks = synth.blocks(g, t, n, k)
    if m >= 8:
        batches = [special_tokens(g, m, k, bf16)]
    else:  # the few-token kernels: every special kind, m tokens per call
        kinds = special_tokens(g, 8, k)[0]
        order = [1, 2, 3, 4, 5, 6, 7, 0]
        sel = [[order[(i + j) % 8] for j in range(m)] for i in range(0, 8, m)]
        batches = [(kinds[s], kinds[s]) for s in sel]
    for xin, xf in batches:
        outs, kernel = _run(backend, t, blocks, n, k, xin, bf16, group)
        assert kernel.startswith(prefix), kernel
        rc, ref = oracle.candle_fused(t, blocks, xf, m, n, k)
        assert rc == 0
        for j, got in enumerate(outs):
            assert_same_class(got, ref.reshape(m, n), f"{kernel} out {j}")


@pytest.mark.gpu
@pytest.mark.parametrize("splits", [None, "4", "tiled"])
def test_attention_nonfinite_scores(backend, monkeypatch, splits):
    """NaN, +Inf and -Inf attention scores (a NaN query head, keys with
    +-Inf elements) on the one-workgroup, split-K and tiled forms."""
    if splits == "tiled":
        monkeypatch.setenv("REALM_ATT_TILED", "1")
    elif splits:
        monkeypatch.setenv("REALM_ATT_SPLITS", splits)
    g = np.random.default_rng(81)
    seq, kv, pos, heads, kvh, hd = 2, 300, 298, 8, 2, 64
    q = g.standard_normal(seq * heads * hd).astype(np.float32)
    k = g.standard_normal(kv * kvh * hd).astype(np.float32)
    v = g.standard_normal(kv * kvh * hd).astype(np.float32)
    q[3 * hd + 5] = np.nan                       # token 0, head 3: every score NaN
    k[(17 * kvh + 0) * hd + 2] = np.inf          # key 17, kv head 0: +-Inf scores
    k[(40 * kvh + 1) * hd + 9] = -np.inf         # key 40, kv head 1
    dq, dk, dv = (backend.alloc(a.nbytes).upload(a) for a in (q, k, v))
    do = backend.alloc(q.nbytes)
    try:
        backend.attention_dev(dq.ptr, dk.ptr, dv.ptr, seq, kv, pos, heads, kvh, hd, do.ptr)
        backend.synchronize()
        got = do.download(np.float32, q.size)
    finally:
        for b in (dq, dk, dv, do):
            b.close()
    want = oa.attention(q, k, v, seq, kv, pos, heads, kvh, hd)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = np.isfinite(want)
    assert rel_l2(got[fin], want[fin]) < 1e-5


Q80_SCALE_CASES = [  # (m, bf16, forced tile, forced K split, kernel)
    (37, False, "t4112p2", "1", "realm_gemm_q80_t4112p2"),
    (37, False, "t4112p2", "4", "realm_gemm_tiled_reduce"),
    (64, True, "t4112b2", "1", "realm_gemm_q80_t4112b2"),
    (64, True, "t4112b2", "2", "realm_gemm_tiled_reduce"),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", Q80_SCALE_CASES, ids=[f"m{c[0]}-{c[2]}-ks{c[3]}" for c in Q80_SCALE_CASES])
def test_q80_tiled_scales(backend, oracle, monkeypatch, case):
    """Q8_0 scales the tiled kernel's f16 (d q) split cannot hold: rows with
    a block scale of magnitude 512 or more, NaN or +-Inf are computed by the
    exact f32 path (direct epilogue, or the reduce after a K split); a row
    whose scale is 511.75 with q = -128 (d q = -65504, the largest f16) stays
    on the MFMA path.  NaN and Inf positions match the oracle's f32 product,
    finite entries within 1e-3 per token."""
    m, bf16, tile, ks, kernel = case
    monkeypatch.setenv("REALM_GEMM_TILE", tile)
    monkeypatch.setenv("REALM_GEMM_KS", ks)
    g = synth.rng(zlib.crc32(repr(case).encode()) % 100000)
    n, k = 200, 2048
    blocks = synth.blocks(g, GGML_Q8_0, n, k)
    blocks["quants"] = g.integers(-128, 128, blocks["quants"].shape, dtype=np.int8)
    kb = k // 32
    f16 = lambda v: np.array([v], np.float16).view(np.uint16)[0]
    blocks["scale"][5 * kb + 3] = f16(600.0)
    blocks["scale"][6 * kb + 40] = f16(-512.0)
    blocks["scale"][7 * kb + 63] = f16(65504.0)
    blocks["scale"][9 * kb + 10] = f16(511.75)
    blocks["quants"][9 * kb + 10] = -128
    blocks["scale"][150 * kb + 2] = f16(np.nan)
    blocks["scale"][151 * kb + 20] = f16(np.inf)
    blocks["scale"][152 * kb + 33] = f16(-np.inf)
    if bf16:
        xb = synth.activations_bf16(g, m, k)
        xin, xf = xb, synth.bf16_bits_to_f32(xb)
    else:
        xin = xf = synth.activations(g, m, k)
    (got,), ran = _run(backend, GGML_Q8_0, blocks, n, k, xin, bf16)
    assert ran == kernel, ran
    rc, ref = oracle.candle_fused(GGML_Q8_0, blocks, xf, m, n, k)
    assert rc == 0
    ref = ref.reshape(m, n)
    assert np.isnan(ref[:, 150]).all() and not np.isfinite(ref[:, 151:153]).any()
    assert_same_class(got, ref, ran)
    for r in (5, 6, 7, 9):  # the planted rows, each on its own
        err = rel_l2(got[:, r], ref[:, r])
        assert err < REL_TOL, f"row {r}: rel_l2 {err:.3e}"

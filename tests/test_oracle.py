"""Pins the CPU oracle (oracle/realm_oracle.c) before anything is compared
with it.  Every check is independent of the oracle's own formulas: golden
known answers from the reference's tests (tests/golden/kat.npz), numpy's own
float16 conversion, an independent packer for the 6-bit scale layout, fp64
brute force, and the invariants the reference's tests assert.
"""
import numpy as np
import pytest

from realm_amd import synth
from realm_amd.formats import GGML_Q4_K, GGML_Q6_K, GGML_Q8_0, Q4K_DTYPE, Q6K_DTYPE, Q80_DTYPE

from conftest import rel_l2


# ------------------------------------------------------------------- f16

def test_f16_to_f32_all_patterns(oracle):
    """All 65536 binary16 patterns against numpy's float16 -> float32."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne(oracle):
    g = np.random.default_rng(7)
    vals = np.concatenate([
        g.standard_normal(20000).astype(np.float32) * np.float32(1e-3),
        g.standard_normal(20000).astype(np.float32) * np.float32(1e4),
        np.array([0.0, -0.0, 65504.0, 65520.0, 1e-8, 2.0 ** -25, 2.0 ** -24, 3 * 2.0 ** -26,
                  np.inf, -np.inf], np.float32)])
    ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, ref)


# ---------------------------------------------------------- scale layout

def pack_scale_min_k4(sc, m):
    """Independent packer for 8 six-bit (scale, min) pairs into 12 bytes:
    pairs 0..3 sit in the low 6 bits of bytes 0..3 (scale) and 4..7 (min);
    pairs 4..7 put their low 4 bits in the nibbles of bytes 8..11 and their
    high 2 bits in the top bits of bytes 0..3 (scale) and 4..7 (min)."""
    s = [0] * 12
    for j in range(4):
        s[j] = sc[j] & 63
        s[j + 4] = m[j] & 63
    for j in range(4, 8):
        s[j + 4] = (sc[j] & 0xF) | ((m[j] & 0xF) << 4)
        s[j - 4] |= (sc[j] >> 4) << 6
        s[j] |= (m[j] >> 4) << 6
    return s


def test_get_scale_min_k4_roundtrip(oracle):
    g = np.random.default_rng(1)
    for _ in range(400):
        sc = g.integers(0, 64, 8).tolist()
        m = g.integers(0, 64, 8).tolist()
        s = pack_scale_min_k4(sc, m)
        for j in range(8):
            assert oracle.get_scale_min_k4(j, s) == (sc[j], m[j])
    # every 6-bit value in every position
    for v in range(64):
        s = pack_scale_min_k4([v] * 8, [63 - v] * 8)
        for j in range(8):
            assert oracle.get_scale_min_k4(j, s) == (v, 63 - v)


# ------------------------------------------------------------ dequant KATs

def test_dequant_kats(oracle, kat):
    for key, t in (("q4k", GGML_Q4_K), ("q6k", GGML_Q6_K), ("q8", GGML_Q8_0)):
        got = oracle.dequantize(t, kat[f"{key}_kat_block"])
        assert np.array_equal(got, kat[f"{key}_kat_expected"]), key


def test_dequant_positions(oracle, kat):
    for key, t, hot, cold in (("q4k", GGML_Q4_K, 15.0, 0.0), ("q6k", GGML_Q6_K, 31.0, -32.0)):
        y = oracle.dequantize(t, kat[f"{key}_pos_blocks"]).reshape(-1, 256)
        idx = kat[f"{key}_pos_index"]
        for b, i in enumerate(idx):
            exp = np.full(256, cold, np.float32)
            exp[i] = hot
            assert np.array_equal(y[b], exp), (key, b, i)


def _fp64_dequant_q4k(blocks):
    """fp64 restatement from the layout statement in make_golden.py, used
    only to bound the f32 rounding of the oracle."""
    out = []
    for b in blocks:
        d = float(np.uint16(b["d"]).view(np.float16))
        dm = float(np.uint16(b["dmin"]).view(np.float16))
        s = b["scales"].tolist()
        y = np.zeros(256)
        for g in range(4):
            for h in range(2):
                j = 2 * g + h
                if j < 4:
                    sc, m = s[j] & 63, s[j + 4] & 63
                else:
                    sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4)
                    m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
                q = b["qs"][32 * g:32 * g + 32]
                q = (q >> 4) if h else (q & 0xF)
                y[64 * g + 32 * h:64 * g + 32 * h + 32] = d * sc * q - dm * m
        out.append(y)
    return np.concatenate(out)


def test_dequant_q4k_vs_fp64(oracle):
    blocks = synth.q4k_blocks(synth.rng(3), 8, 1024)
    got = oracle.dequantize(GGML_Q4_K, blocks).astype(np.float64)
    ref = _fp64_dequant_q4k(blocks)
    # one f32 rounding of the subtraction at most
    assert np.all(np.abs(got - ref) <= 2.0 ** -23 * np.maximum(np.abs(ref), 1e-30) + 1e-30)


def test_dequant_q6k_q80_exact_products(oracle):
    """Q6_K and Q8_0 outputs are exact products (<= 24 significant bits)."""
    g = synth.rng(4)
    b6 = synth.q6k_blocks(g, 4, 512)
    y = oracle.dequantize(GGML_Q6_K, b6).reshape(-1, 256)
    for i, b in enumerate(b6):
        d = float(np.uint16(b["d"]).view(np.float16))
        ql, qh, sc = b["ql"].astype(int), b["qh"].astype(int), b["scales"].astype(int)
        for h in range(2):
            for l in range(32):
                for t in range(4):
                    lo = ql[64 * h + l + (32 if t & 1 else 0)]
                    lo = (lo >> 4) if t & 2 else (lo & 0xF)
                    q = (lo | (((qh[32 * h + l] >> (2 * t)) & 3) << 4)) - 32
                    assert y[i, 128 * h + l + 32 * t] == d * sc[8 * h + l // 16 + 2 * t] * q
    b8 = synth.q80_blocks(g, 4, 64)
    y8 = oracle.dequantize(GGML_Q8_0, b8).reshape(-1, 32)
    d8 = b8["scale"].view(np.float16).astype(np.float64)
    assert np.array_equal(y8, (b8["quants"].astype(np.float64) * d8[:, None]).astype(np.float32))


def test_dequantize_tensor_validation(oracle):
    blocks = synth.q4k_blocks(synth.rng(5), 2, 256)
    raw = blocks.view(np.uint8)
    rc, _ = oracle.dequantize_tensor(GGML_Q4_K, raw[:-1], 512)
    assert rc == oracle.MODEL_PARSE_ERROR
    rc, _ = oracle.dequantize_tensor(GGML_Q4_K, raw, 500)
    assert rc == oracle.INVALID_ARGUMENT
    b6 = synth.q6k_blocks(synth.rng(6), 2, 256).view(np.uint8)
    rc, y = oracle.dequantize_tensor(GGML_Q6_K, np.concatenate([b6, b6[:50]]), 600)
    assert rc == oracle.OK and np.all(y[512:] == 0)  # partial block ignored, tail zero
    rc, _ = oracle.dequantize_tensor(GGML_Q6_K, b6, 300)
    assert rc == oracle.PANIC


# ------------------------------------------------------------------ fused

def _ref_test_q4k_blocks():
    """fused.rs:2848-2861 inputs (N=2, K=512)."""
    b = np.zeros(4, Q4K_DTYPE)
    for i in range(2):
        for j in range(2):
            e = b[2 * i + j]
            e["d"] = np.float16(0.5 + i * 0.1).view(np.uint16)
            e["dmin"] = np.float16(0.1).view(np.uint16)
            e["scales"] = 16 + i + j
            e["qs"] = (i * 17 + j * 13) % 256
    return b


def _ref_test_q6k_blocks():
    """fused.rs:3491-3517 inputs."""
    b = np.zeros(4, Q6K_DTYPE)
    for i in range(2):
        for j in range(2):
            e = b[2 * i + j]
            e["ql"] = [(i * 15 + j * 9 + t) % 255 for t in range(128)]
            e["qh"] = [(i * 13 + j * 7 + t) % 255 for t in range(64)]
            e["scales"] = [((i * 9 + j * 5 + t) % 127) - 64 for t in range(16)]
            e["d"] = np.float16(0.5 + i * 0.1).view(np.uint16)
    return b


def _ref_test_q80_blocks():
    """fused.rs:3656-3670 inputs (K=64)."""
    b = np.zeros(4, Q80_DTYPE)
    for i in range(2):
        for j in range(2):
            e = b[2 * i + j]
            e["quants"] = [((i * 13 + j * 7 + t) % 127) - 64 for t in range(32)]
            e["scale"] = np.float16(0.5 + i * 0.1).view(np.uint16)
    return b


@pytest.mark.parametrize("t,k,mk", [(GGML_Q4_K, 512, _ref_test_q4k_blocks),
                                    (GGML_Q6_K, 512, _ref_test_q6k_blocks),
                                    (GGML_Q8_0, 64, _ref_test_q80_blocks)])
def test_fused_matches_dequant_dot(oracle, t, k, mk):
    """The reference's own invariant (fused.rs:2839-2915, 3482-3572,
    3647-3726): fused == dequantize + dot within rel 1e-4."""
    blocks = mk()
    x = ((np.arange(k) % 7).astype(np.float32) - 3.0) * 0.5
    rc, fused = oracle.fused(t, blocks, x, 1, 2, k)
    assert rc == 0
    w = oracle.dequantize(t, blocks).reshape(2, k)
    ref = w.astype(np.float64) @ x.astype(np.float64)
    for i in range(2):
        assert abs(fused[i] - ref[i]) <= 1e-4 * max(abs(ref[i]), 1e-6)


@pytest.mark.parametrize("t", [GGML_Q4_K, GGML_Q6_K, GGML_Q8_0])
def test_fused_and_candle_vs_fp64(oracle, t):
    g = synth.rng(11)
    n, k, batch = 48, 1024, 3
    blocks = synth.blocks(g, t, n, k)
    x = synth.activations(g, batch, k)
    w = oracle.dequantize(t, blocks)
    ref = oracle.matvec_f64(w, x, batch, n, k)
    rc, fz = oracle.fused(t, blocks, x, batch, n, k)
    assert rc == 0 and rel_l2(fz, ref) < 1e-5
    rc, cz = oracle.candle_fused(t, blocks, x, batch, n, k)
    assert rc == 0 and rel_l2(cz, ref) < 1e-5
    # the brute force itself: numpy float64 matmul of the same dequantized W
    assert rel_l2(ref, (x.astype(np.float64) @ w.reshape(n, k).astype(np.float64).T).ravel()) < 1e-12


def test_fused_validation(oracle):
    """fused.rs:2977-3000 and webgpu_dequant_tests.rs:238-298."""
    one = np.zeros(1, Q4K_DTYPE)
    rc, _ = oracle.fused(GGML_Q4_K, one, np.zeros(256, np.float32), 1, 1, 100)
    assert rc == oracle.INVALID_ARGUMENT
    rc, _ = oracle.fused(GGML_Q4_K, one, np.zeros(256, np.float32), 1, 2, 256)
    assert rc == oracle.INVALID_ARGUMENT
    rc, _ = oracle.fused(GGML_Q8_0, np.zeros(2, Q80_DTYPE), np.zeros(60, np.float32), 1, 1, 64)
    assert rc == oracle.INVALID_ARGUMENT


def test_q80_tail_quirk(oracle):
    """K % 32 != 0: ceil(n*k/32) blocks, per-row stride ceil(k/32); block
    indices past the end are skipped (fused.rs:2459, 2484-2500)."""
    n, k = 2, 40  # 3 blocks expected, rows use blocks (0,1) and (2,<missing>)
    b = np.zeros(3, Q80_DTYPE)
    b["scale"] = np.float16(1.0).view(np.uint16)
    b["quants"] = 1
    x = np.ones(k, np.float32)
    rc, y = oracle.fused(GGML_Q8_0, b, x, 1, n, k)
    assert rc == 0
    assert y[0] == 40.0 and y[1] == 32.0


def test_nan_scale_fallback(oracle):
    """fused.rs:276-285: a NaN d becomes 6e-8 in fused.rs; the dequantizer
    (and so CandleCpuBackend) propagates NaN."""
    b = synth.q4k_blocks(synth.rng(2), 1, 256)
    b["d"] = 0x7E00
    x = np.ones(256, np.float32)
    rc, y = oracle.fused(GGML_Q4_K, b, x, 1, 1, 256, nan_fallback=True)
    assert rc == 0 and np.isfinite(y).all()
    rc, y2 = oracle.candle_fused(GGML_Q4_K, b, x, 1, 1, 256)
    assert rc == 0 and np.isnan(y2).all()
    rc, y3 = oracle.fused(GGML_Q4_K, b, x, 1, 1, 256, nan_fallback=False)
    assert np.isnan(y3).all()


# ------------------------------------------------------------------ dense

def test_dense_kats(oracle, kat):
    rc, c = oracle.matmul_f32(kat["dense_a1"], kat["dense_b1"], 2, 3, 2)
    assert rc == 0 and np.array_equal(c, kat["dense_e1"])
    rc, c = oracle.matmul_transposed(kat["dense_a2"], kat["dense_bt2"], 2, 2, 2)
    assert rc == 0 and np.array_equal(c, kat["dense_e2"])
    rc, c = oracle.matmul_f32(kat["dense_a3"], kat["dense_b3"], 2, 2, 2)
    assert rc == 0 and np.array_equal(c, kat["dense_e3"])
    rc, _ = oracle.matmul_f32(kat["dense_a1"], kat["dense_b1"], 2, 2, 2)
    assert rc == oracle.INVALID_ARGUMENT


# ------------------------------------------------------------------- LoRA

def test_lora_kats(oracle, kat):
    rc, out = oracle.lora_apply_to_weights(np.ones(16), np.full(8, 0.5), np.full(8, 0.5),
                                           2, 4.0, 4, 4)
    assert rc == 0 and np.array_equal(out, kat["lora1_expected"])
    rc, out = oracle.lora_apply_to_weights(np.ones(16), np.full(16, 0.1), np.full(16, 0.2),
                                           4, 8.0, 4, 4)
    assert rc == 0 and np.array_equal(out, kat["lora2_expected"])


def test_lora_merged_equals_unmerged(oracle):
    """(W + s B A) x == W x + s B (A x) up to f32 rounding; id -1 leaves the
    base output untouched."""
    g = synth.rng(9)
    n, k, m = 64, 256, 6
    blocks = synth.q4k_blocks(g, n, k)
    w = oracle.dequantize(GGML_Q4_K, blocks)
    x = synth.activations(g, m, k)
    adapters = []
    for r in (4, 8):
        a, b = synth.lora_adapter(g, r, k, n)
        adapters.append((a.astype(np.float32), b.astype(np.float32), r, 16.0))
    ids = np.array([0, 1, -1, 1, 0, 5], np.int32)
    rc, base = oracle.matmul_transposed(x, w, m, k, n)
    y = oracle.multi_lora_delta(x, ids, adapters, base.reshape(m, n).copy())
    for t in range(m):
        a = ids[t]
        if a < 0 or a >= len(adapters):
            assert np.array_equal(y[t], base.reshape(m, n)[t])
            continue
        A, B, r, al = adapters[a]
        rc, wm = oracle.lora_apply_to_weights(w, A, B, r, al, n, k)
        rc, ym = oracle.matmul_transposed(x[t], wm, 1, k, n)
        assert rel_l2(y[t], ym) < 1e-5

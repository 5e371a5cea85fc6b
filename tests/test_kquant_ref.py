"""The reference's own 256-element Q2_K, Q3_K, Q5_K and Q8_K layouts
(crates/realm-core/src/quant.rs:71-95, 200-222; #[repr(C)] sizes 116, 196,
178 and 292 bytes, which are not ggml's) and their dequantizers
(quant.rs:453-638), plus the Q5_0 / Q5_1 high-bit map.

CPU: the oracle against known answers written down by hand
(tests/golden/make_golden.py): the inputs of the reference's own Q5_K / Q8_K
tests with their closed-form outputs, one-hot probes of every element's bits,
and the scale maps.  GPU: the device dequantization bit-exact with the oracle
on random blocks and on those fixtures, and the fused products (CandleGpuBackend
semantics, candle_backend.rs:507-571, 639-836) within 1e-3 relative L2, as
one-call trait products and as registered resident weights."""
import numpy as np
import pytest

from conftest import rel_l2

Q2K, Q3K, Q5K, Q8K = 10, 11, 13, 15
BB = {Q2K: 116, Q3K: 196, Q5K: 178, Q8K: 292}
FN = {Q2K: "q2k", Q3K: "q3k", Q5K: "q5k", Q8K: "q8k"}


def _deq(oracle, t, raw):
    rc, y = oracle.dequantize_tensor(t, raw, raw.size // BB[t] * 256)
    assert rc == 0
    return y


def _random_blocks(t, nb, seed):
    g = np.random.default_rng(seed)
    raw = g.integers(0, 256, (nb, BB[t]), dtype=np.uint8)
    # scales d / dmin: finite f16 around 1e-2 (random bytes would include
    # Inf and NaN patterns; those are covered by the exact fixtures' d = 1)
    dpos = {Q2K: 0, Q3K: 0, Q5K: 176, Q8K: 288}[t]
    for off in ((dpos,) if t == Q5K else (dpos, dpos + 2)):
        h = (np.abs(g.standard_normal(nb)) * 1e-2).astype(np.float16).view(np.uint16)
        raw[:, off] = h & 0xFF
        raw[:, off + 1] = h >> 8
    return raw.reshape(-1)


# ----------------------------------------------------------------- CPU

def test_oracle_reference_test_inputs(oracle, kat):
    assert np.array_equal(_deq(oracle, Q5K, kat["q5k_kat_block"]), kat["q5k_kat_expected"])
    assert np.array_equal(_deq(oracle, Q8K, kat["q8k_kat_block"]), kat["q8k_kat_expected"])


@pytest.mark.parametrize("key,t", [("q2k_pos", Q2K), ("q3k_pos", Q3K), ("q5k_pos", Q5K),
                                   ("q2k_scale", Q2K), ("q3k_scale", Q3K), ("q8k_scale", Q8K)])
def test_oracle_probes(oracle, kat, key, t):
    raw = kat[key + ("_blocks" if key.endswith("pos") else "_block")]
    assert np.array_equal(_deq(oracle, t, raw), kat[key + "_expected"]), key


@pytest.mark.parametrize("t,key", [(6, "q5_0"), (7, "q5_1")])
def test_oracle_q5_high_bit_map(oracle, kat, t, key):
    raw = kat[f"{key}_qh_blocks"]
    rc, y = oracle.dequantize_tensor(t, raw, raw.size // (22 if t == 6 else 24) * 32)
    assert rc == 0 and np.array_equal(y, kat[f"{key}_qh_expected"]), key


def test_oracle_q5k_upper_half_zero(oracle):
    """Q5_K: the reference writes elements 0..127 only, whatever the bytes."""
    y = _deq(oracle, Q5K, _random_blocks(Q5K, 8, 1)).reshape(8, 256)
    assert np.all(y[:, 128:] == 0) and np.any(y[:, :128] != 0)


def test_oracle_fused_equals_dequant_dot(oracle):
    """CandleCpuBackend semantics: the fused product is the dequantized
    matrix times x (fp64 check of the oracle's f32 sums)."""
    g = np.random.default_rng(3)
    for t in (Q2K, Q3K, Q5K, Q8K):
        n, k, m = 12, 512, 3
        raw = _random_blocks(t, n * k // 256, 10 + t)
        x = g.standard_normal((m, k)).astype(np.float32)
        rc, y = oracle.candle_fused(t, raw, x, m, n, k)
        assert rc == 0
        w = _deq(oracle, t, raw).reshape(n, k).astype(np.float64)
        assert rel_l2(y.reshape(m, n), x.astype(np.float64) @ w.T) < 1e-6, t


# ----------------------------------------------------------------- GPU

@pytest.mark.gpu
@pytest.mark.parametrize("t", [Q2K, Q3K, Q5K, Q8K])
def test_dequant_bit_exact(backend, oracle, kat, t):
    raw = _random_blocks(t, 333, 20 + t)
    got = backend.dequantize(t, raw, 333 * 256)
    ref = _deq(oracle, t, raw)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    for key in [k for k in kat if k.startswith(FN[t]) and k.endswith(("_blocks", "_block"))]:
        want = kat[key.rsplit("_", 1)[0] + "_expected"]
        assert np.array_equal(backend.dequantize(t, kat[key], want.size), want), key


@pytest.mark.gpu
@pytest.mark.parametrize("t", [6, 7])
def test_q5_high_bit_map_device(backend, kat, t):
    key = "q5_0" if t == 6 else "q5_1"
    want = kat[f"{key}_qh_expected"]
    assert np.array_equal(backend.dequantize(t, kat[f"{key}_qh_blocks"], want.size), want)


@pytest.mark.gpu
@pytest.mark.parametrize("t", [Q2K, Q3K, Q5K, Q8K])
@pytest.mark.parametrize("m", [1, 5, 40])
def test_fused_products(backend, oracle, t, m):
    g = np.random.default_rng(30 + t + m)
    n, k = 96, 1024
    raw = _random_blocks(t, n * k // 256, 40 + t + m)
    x = g.standard_normal((m, k)).astype(np.float32)
    got = getattr(backend, f"fused_dequant_matmul_{FN[t]}")(raw, x, m, n, k)
    rc, ref = oracle.candle_fused(t, raw, x, m, n, k)
    assert rc == 0 and rel_l2(got, ref) < 1e-3, t
    # resident weights: registered once, kept dequantized
    h = backend.register_weights(t, raw, n, k)
    try:
        assert rel_l2(backend.weights_matmul(h, x), ref) < 1e-3
    finally:
        backend.release_weights(h)


@pytest.mark.gpu
def test_validation(backend):
    from realm_amd.backend import InvalidShape, RealmError
    raw = np.zeros(BB[Q5K] * 2, np.uint8)
    with pytest.raises(InvalidShape):  # k not a multiple of 256
        backend.fused_dequant_matmul_q5k(raw, np.zeros(300, np.float32), 1, 1, 300)
    with pytest.raises(InvalidShape):  # block count
        backend.fused_dequant_matmul_q5k(raw, np.zeros(256, np.float32), 1, 1, 256)
    with pytest.raises(RealmError) as e:  # input length: the tensor creation fails
        backend.fused_dequant_matmul_q5k(raw, np.zeros(500, np.float32), 1, 2, 256)
    assert e.value.code == 1

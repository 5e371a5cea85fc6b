"""The reference's 32-element block formats Q4_0, Q4_1, Q5_0, Q5_1, Q8_1
(crates/realm-core/src/quant.rs:10-70, 226-370): the oracle pinned by closed
forms (CPU), the HIP dequantization bit-exact against it and the fused
dequant x matmul (CandleGpuBackend semantics) within 1e-3 relative L2 (GPU).

Which qh bit feeds which Q5_0 / Q5_1 element is the reference's own index
formula (quant.rs:283-350; it matches neither ggml nor any reference test);
the checks below pin the low nibbles and that a set high bit adds 16, and the
bit-to-element map is pinned by hand-written one-hot tables
(tests/golden/make_golden.py, checked in tests/test_kquant_ref.py)."""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import oracle as o

BB = {2: 18, 3: 20, 6: 22, 7: 24, 9: 36}
NAME = {2: "q40", 3: "q41", 6: "q50", 7: "q51", 9: "q81"}
HALF_ONE, HALF_TWO, HALF_QUARTER = 0x3C00, 0x4000, 0x3400


def _block(t, scale=HALF_ONE, delta=0, fill=0, qh=0):
    b = bytearray(BB[t])
    b[0:2] = scale.to_bytes(2, "little")
    off = 2
    if t in (3, 7, 9):
        b[2:4] = delta.to_bytes(2, "little")
        off = 4
    if t in (6, 7):
        b[off:off + 4] = bytes([qh] * 4)
        off += 4
    for i in range(off, BB[t]):
        b[i] = fill
    return np.frombuffer(bytes(b), np.uint8)


def _deq(oracle, t, raw):
    rc, y = oracle.dequantize_tensor(t, raw, raw.size // BB[t] * 32)
    assert rc == 0
    return y


def test_oracle_closed_forms(oracle):
    y = _deq(oracle, 2, _block(2, fill=0x80))          # lo 0 -> -8, hi 8 -> 0
    assert np.array_equal(y, np.r_[np.full(16, -8.0), np.zeros(16)])
    y = _deq(oracle, 2, _block(2, scale=HALF_TWO, fill=0x1F))  # lo 15 -> 7, hi 1 -> -7
    assert np.array_equal(y, np.r_[np.full(16, 14.0), np.full(16, -14.0)])
    y = _deq(oracle, 3, _block(3, delta=HALF_QUARTER, fill=0x80))
    assert np.array_equal(y, np.r_[np.full(16, -7.75), np.full(16, 0.25)])
    y = _deq(oracle, 9, _block(9, scale=HALF_TWO, delta=HALF_QUARTER, fill=0xFD))  # q = -3
    assert np.array_equal(y, np.full(32, -5.75))
    for t in (6, 7):
        # low nibbles 0x21: even elements 1, odd 2; no high bits -> q - 16
        y = _deq(oracle, t, _block(t, fill=0x21, qh=0x00))
        assert np.array_equal(y, np.tile([-15.0, -14.0], 16)), t
        # every high bit set: each element gets +16 whatever its bit
        y = _deq(oracle, t, _block(t, fill=0x21, qh=0xFF))
        assert np.array_equal(y, np.tile([1.0, 2.0], 16)), t


def _random_blocks(g, t, nb, special=False):
    raw = g.integers(0, 256, nb * BB[t], dtype=np.uint8).reshape(nb, BB[t])
    scale = (np.abs(g.standard_normal(nb)) * 1e-2).astype(np.float16).view(np.uint8)
    raw[:, 0:2] = scale.reshape(nb, 2)
    if t in (3, 7, 9):
        raw[:, 2:4] = (g.standard_normal(nb) * 1e-2).astype(np.float16).view(np.uint8).reshape(nb, 2)
    if special:
        specials = np.array([0x0001, 0x8000, 0x7BFF, 0x7C00, 0xFC00, 0x7E00, 0x0000], np.uint16)
        raw[:len(specials), 0:2] = specials.view(np.uint8).reshape(-1, 2)
    return raw.reshape(-1)


@pytest.mark.gpu
@pytest.mark.parametrize("t", [2, 3, 6, 7, 9])
def test_dequant_bit_exact(backend, oracle, t):
    g = np.random.default_rng(t)
    raw = _random_blocks(g, t, 4096, special=True)
    got = backend.dequantize(t, raw, 4096 * 32)
    want = _deq(oracle, t, raw)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # dequantize_tensor: trailing partial block ignored, tail zero-filled
    got = backend.dequantize(t, raw[:3 * BB[t] + 5], 100)
    rc, want = oracle.dequantize_tensor(t, raw[:3 * BB[t] + 5], 100)
    assert rc == 0 and np.array_equal(got[:96].view(np.uint32), want[:96].view(np.uint32))
    assert np.array_equal(got[96:], np.zeros(4, np.float32))


@pytest.mark.gpu
@pytest.mark.parametrize("t", [2, 3, 6, 7, 9])
@pytest.mark.parametrize("m,n,k", [(1, 70, 256), (5, 33, 96), (33, 300, 1024)])
def test_fused(backend, oracle, t, m, n, k):
    g = np.random.default_rng(100 * t + m)
    raw = _random_blocks(g, t, n * k // 32)
    x = g.standard_normal(m * k).astype(np.float32)
    got = getattr(backend, f"fused_dequant_matmul_{NAME[t]}")(raw, x, m, n, k)
    rc, want = oracle.candle_fused(t, raw, x, m, n, k)
    assert rc == 0
    err = rel_l2(got, want)
    print(f"{NAME[t]} m={m} n={n} k={k} rel_l2={err:.3e}")
    assert err < 1e-3


@pytest.mark.gpu
def test_fused_validation(backend):
    from realm_amd.backend import InvalidShape
    raw = np.zeros(18 * 4, np.uint8)
    with pytest.raises(InvalidShape):   # k % 32
        backend.fused_dequant_matmul_q40(raw, np.zeros(40, np.float32), 1, 1, 40)
    with pytest.raises(InvalidShape):   # block count
        backend.fused_dequant_matmul_q40(raw, np.zeros(64, np.float32), 1, 1, 64)
    with pytest.raises(InvalidShape):   # input length
        backend.fused_dequant_matmul_q40(raw, np.zeros(63, np.float32), 1, 2, 64)


@pytest.mark.gpu
@pytest.mark.parametrize("t", [2, 3, 6, 7, 9])
@pytest.mark.parametrize("n,k", [(96, 512), (200, 4128)])
def test_resident_weights(backend, oracle, t, n, k):
    """Registered once (repacked as int8 q', f16 scale, f16 delta: 1.125
    bytes per weight), then products at 1-4 tokens (int8-dot GEMV), 7 and 20
    (4 tokens per GEMV launch) and 50 (dequantized bit-exactly into the
    workspace, dense f32 GEMM), alone and in a grouped call, against the
    oracle; K = 4128 is not a multiple of 64 (padded layout); LoRA on such a
    base is refused."""
    from realm_amd.backend import BackendError
    g = np.random.default_rng(500 + t + n)
    raw = _random_blocks(g, t, n * k // 32)
    h = backend.register_weights(t, raw, n, k)
    h2 = backend.register_weights(t, raw, n, k)
    try:
        for m in (1, 2, 3, 4, 7, 20, 50):
            x = g.standard_normal(m * k).astype(np.float32)
            got = backend.weights_matmul(h, x.reshape(m, k))
            kern = backend.last_kernel()
            assert kern.startswith("realm_gemv_q8m" if m <= 48 else "realm_dense"), (m, kern)
            rc, want = oracle.candle_fused(t, raw, x, m, n, k)
            assert rc == 0 and rel_l2(got, want.reshape(m, n)) < 1e-3, m
            dx = backend.alloc(x.nbytes).upload(x)
            dys = [backend.alloc(m * n * 4) for _ in range(2)]
            backend.matmul_group_dev([h, h2], dx.ptr, m, [d.ptr for d in dys])
            backend.synchronize()
            for d in dys:
                assert rel_l2(d.download(np.float32, m * n), want) < 1e-3
            for b in dys + [dx]:
                b.close()
        a = (g.standard_normal((8, k)) * 0.01).astype(np.float32)
        b = (g.standard_normal((n, 8)) * 0.01).astype(np.float32)
        ah = backend.lora_register(a, b, 8, 16.0, k, n)
        sh = backend.lora_set_create([ah])
        with pytest.raises(BackendError):
            backend.multi_lora_matmul(h, sh, g.standard_normal((2, k)).astype(np.float32),
                                      np.zeros(2, np.int32))
        backend.lora_set_release(sh)
        backend.lora_release(ah)
    finally:
        backend.release_weights(h)
        backend.release_weights(h2)

"""GPU parity: the HIP path through the C ABI against the CPU oracle on the
same seeded inputs.

Bars: dequantization is bit-exact with quant.rs; matmul and LoRA outputs
agree with realm-compute-cpu's CandleCpuBackend semantics (dequantize, then
f32 x . W^T) within 1e-3 relative L2 error (REL_TOL, the tolerance of the
workload definition).  Full-size configurations are compared on the full
output where the oracle finishes in seconds, otherwise on a seeded subset of
rows.
"""
import zlib

import numpy as np
import pytest

from realm_amd import synth
from realm_amd.backend import BackendError, InvalidShape, RealmError
from realm_amd.formats import GGML_Q4_K, GGML_Q6_K, GGML_Q8_0, NAMES, Q4K_DTYPE, Q6K_DTYPE
from realm_amd.formats import Q80_DTYPE

from conftest import rel_l2

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3
FORMATS = [GGML_Q4_K, GGML_Q6_K, GGML_Q8_0]


def bits_equal(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(b)
    return np.array_equal(np.isnan(a), nan) and np.array_equal(a[~nan].view(np.uint32),
                                                               b[~nan].view(np.uint32))


def special_scales(g, blocks, field):
    """Overwrite some f16 scales with edge values: subnormals, -0, max, inf, nan."""
    v = blocks[field]
    n = v.size
    pick = g.choice(n, size=min(n, 64), replace=False)
    specials = np.array([0x0001, 0x03FF, 0x0200, 0x8000, 0x8001, 0x7BFF, 0xFBFF, 0x7C00,
                         0xFC00, 0x7E00, 0x3C00, 0x0000], np.uint16)
    v[pick] = specials[np.arange(pick.size) % specials.size]


# ---------------------------------------------------------------- basics

def test_init_and_name(backend):
    assert "gfx950" in backend.name()


@pytest.mark.parametrize("t", FORMATS)
def test_dequant_bit_exact(backend, oracle, t):
    g = synth.rng(100 + t)
    blocks = synth.blocks(g, t, 64, 4096)
    special_scales(g, blocks, "scale" if t == GGML_Q8_0 else "d")
    if t == GGML_Q4_K:
        special_scales(g, blocks, "dmin")
    n_el = blocks.size * (32 if t == GGML_Q8_0 else 256)
    got = backend.dequantize(t, blocks, n_el)
    ref = oracle.dequantize(t, blocks)
    assert bits_equal(got, ref)


def test_dequant_kats_and_positions(backend, kat):
    for key, t in (("q4k", GGML_Q4_K), ("q6k", GGML_Q6_K), ("q8", GGML_Q8_0)):
        blk = kat[f"{key}_kat_block"]
        exp = kat[f"{key}_kat_expected"]
        assert bits_equal(backend.dequantize(t, blk, exp.size), exp), key
    for key, t, hot, cold in (("q4k", GGML_Q4_K, 15.0, 0.0), ("q6k", GGML_Q6_K, 31.0, -32.0)):
        blocks = kat[f"{key}_pos_blocks"]
        idx = kat[f"{key}_pos_index"]
        y = backend.dequantize(t, blocks, idx.size * 256).reshape(-1, 256)
        exp = np.full_like(y, cold)
        exp[np.arange(idx.size), idx] = hot
        assert np.array_equal(y, exp), key


def test_dequantize_tensor_semantics(backend, oracle):
    b4 = synth.q4k_blocks(synth.rng(5), 2, 256).view(np.uint8)
    with pytest.raises(RealmError) as e:
        backend.dequantize(GGML_Q4_K, b4[:-1], 512)
    assert e.value.code == 4  # ModelParseError (Error::InvalidFormat)
    with pytest.raises(InvalidShape):
        backend.dequantize(GGML_Q4_K, b4, 500)
    b6 = synth.q6k_blocks(synth.rng(6), 2, 256).view(np.uint8)
    raw = np.concatenate([b6, b6[:50]])
    got = backend.dequantize(GGML_Q6_K, raw, 600)
    rc, ref = oracle.dequantize_tensor(GGML_Q6_K, raw, 600)
    assert rc == 0 and bits_equal(got, ref)
    with pytest.raises(InvalidShape):  # the reference panics here
        backend.dequantize(GGML_Q6_K, b6, 300)
    with pytest.raises(BackendError):
        backend.dequantize(1, b6, 256)  # F16: not a block format of this path


def test_trait_validation(backend):
    """fused.rs:2977-3000 / webgpu_dequant_tests.rs:238-333 error cases."""
    one = np.zeros(1, Q4K_DTYPE)
    with pytest.raises(InvalidShape):
        backend.fused_dequant_matmul_q4k(one, np.zeros(100, np.float32), 1, 1, 100)
    with pytest.raises(InvalidShape):
        backend.fused_dequant_matmul_q4k(one, np.zeros(256, np.float32), 1, 2, 256)
    with pytest.raises(InvalidShape):  # wrong input length
        backend.fused_dequant_matmul_q4k(np.zeros(4, Q4K_DTYPE), np.zeros(255, np.float32),
                                         1, 4, 256)
    with pytest.raises(InvalidShape):
        backend.fused_dequant_matmul_q80(np.zeros(2, Q80_DTYPE), np.zeros(40, np.float32),
                                         1, 1, 40)
    # a type the backend does not build (F16 here): a cheap BackendUnsupported,
    # so dispatch_matmul falls back to the CPU
    x = np.zeros(256, np.float32)
    out = np.zeros(1, np.float32)
    rc = backend.lib.realm_hip_fused_dequant_matmul(1, x.ctypes.data, 1, x.ctypes.data, 256, 1, 1,
                                                    256, out.ctypes.data)
    assert rc == 5, rc
    # empty K: zero output, like the reference's empty accumulation
    y = backend.fused_dequant_matmul_q4k(np.zeros(0, Q4K_DTYPE), np.zeros(0, np.float32), 2, 3, 0)
    assert np.array_equal(y, np.zeros(6, np.float32))


# ---------------------------------------------------------------- matmul

def test_fused_reference_inputs(backend, oracle):
    """The reference's own fused.rs test inputs (N=2)."""
    from test_oracle import _ref_test_q4k_blocks, _ref_test_q6k_blocks, _ref_test_q80_blocks
    for t, k, mk in ((GGML_Q4_K, 512, _ref_test_q4k_blocks), (GGML_Q6_K, 512, _ref_test_q6k_blocks),
                     (GGML_Q8_0, 64, _ref_test_q80_blocks)):
        blocks = mk()
        x = ((np.arange(k) % 7).astype(np.float32) - 3.0) * 0.5
        got = backend._fused(t, blocks, x, 1, 2, k)
        rc, ref = oracle.candle_fused(t, blocks, x, 1, 2, k)
        assert rc == 0 and rel_l2(got, ref) < REL_TOL, NAMES[t]


@pytest.mark.parametrize("t", FORMATS)
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 16, 17, 33, 64, 100, 130])
def test_fused_random(backend, oracle, t, m):
    g = synth.rng(1000 * t + m)
    n, k = 200, 1024 if t != GGML_Q8_0 else 1056
    blocks = synth.blocks(g, t, n, k)
    x = synth.activations(g, m, k)
    got = backend._fused(t, blocks, x, m, n, k)
    rc, ref = oracle.candle_fused(t, blocks, x, m, n, k)
    assert rc == 0
    err = rel_l2(got, ref)
    print(f"{NAMES[t]} m={m} rel_l2={err:.3e}")
    assert err < REL_TOL


@pytest.mark.parametrize("t", FORMATS)
def test_fused_odd_shapes(backend, oracle, t):
    """Short rows (K = one block), N not a multiple of any tile."""
    g = synth.rng(77 + t)
    for n, k, m in ((1, 256, 1), (3, 256, 3), (17, 512, 1), (129, 768, 19)):
        if t == GGML_Q8_0:
            k = k // 8 * 3 if k > 256 else 96  # K % 64 != 0 exercises the padded layout
        blocks = synth.blocks(g, t, n, k)
        x = synth.activations(g, m, k)
        got = backend._fused(t, blocks, x, m, n, k)
        rc, ref = oracle.candle_fused(t, blocks, x, m, n, k)
        assert rc == 0 and rel_l2(got, ref) < REL_TOL, (n, k, m)


def test_config0_full(backend, oracle):
    """Q4_K GEMV M=1, W 5632 x 2048 (the reference's CPU-runnable case)."""
    g = synth.rng(0)
    n, k = 5632, 2048
    blocks = synth.q4k_blocks(g, n, k)
    x = synth.activations(g, 1, k)
    h = backend.register_weights(GGML_Q4_K, blocks, n, k)
    try:
        got = backend.weights_matmul(h, x)
    finally:
        backend.release_weights(h)
    rc, ref = oracle.candle_fused(GGML_Q4_K, blocks, x, 1, n, k)
    assert rc == 0 and rel_l2(got, ref) < REL_TOL


LAYER_7B = [("wq", GGML_Q4_K, 4096, 4096), ("wk", GGML_Q4_K, 4096, 4096),
            ("wv", GGML_Q4_K, 4096, 4096), ("wo", GGML_Q4_K, 4096, 4096),
            ("w_gate", GGML_Q4_K, 11008, 4096), ("w_up", GGML_Q4_K, 11008, 4096),
            ("w_down", GGML_Q6_K, 4096, 11008)]


@pytest.mark.parametrize("m", [1, 4, 16])
def test_config1_layer(backend, oracle, m):
    """The LLaMA-7B decoder-layer matvec set at decode batch 1/4/16."""
    g = synth.rng(1)
    for name, t, n, k in LAYER_7B:
        blocks = synth.blocks(g, t, n, k)
        x = synth.activations(g, m, k)
        h = backend.register_weights(t, blocks, n, k)
        try:
            got = backend.weights_matmul(h, x)
        finally:
            backend.release_weights(h)
        rc, ref = oracle.candle_fused(t, blocks, x, m, n, k)
        err = rel_l2(got, ref)
        print(f"{name} m={m} rel_l2={err:.3e}")
        assert rc == 0 and err < REL_TOL, name


def _row_subset(t, blocks, n, k, rows):
    bpr = k // (32 if t == GGML_Q8_0 else 256)
    return blocks.reshape(n, bpr)[rows].reshape(-1)


@pytest.mark.parametrize("t", [GGML_Q4_K, GGML_Q8_0])
def test_config2_prefill_bf16(backend, oracle, t):
    """Prefill M=512, K=4096 -> N=11008 with bf16 activations (the launch
    bench.py times: the LDS-tiled MFMA kernel for both formats), checked on
    a seeded subset of 96 output rows for all 512 tokens."""
    g = synth.rng(2)
    m, n, k = 512, 11008, 4096
    blocks = synth.blocks(g, t, n, k)
    xb = synth.activations_bf16(g, m, k)
    h = backend.register_weights(t, blocks, n, k)
    dx = backend.alloc(xb.nbytes).upload(xb)
    dy = backend.alloc(m * n * 4)
    try:
        backend.matmul_dev(h, dx.ptr, m, dy.ptr, bf16=True)
        backend.synchronize()
        ran = backend.last_kernel()
        got = dy.download(np.float32, m * n).reshape(m, n)
    finally:
        backend.release_weights(h)
        dx.close()
        dy.close()
    rows = np.sort(synth.rng(22).choice(n, 96, replace=False))
    rc, ref = oracle.candle_fused(t, _row_subset(t, blocks, n, k, rows),
                                  synth.bf16_bits_to_f32(xb), m, rows.size, k)
    assert rc == 0
    err = rel_l2(got[:, rows], ref.reshape(m, rows.size))
    print(f"prefill {NAMES[t]} {ran} rel_l2={err:.3e}")
    assert ran == f"realm_gemm_{'q4k' if t == GGML_Q4_K else 'q80'}_t4112b2", ran
    assert err < REL_TOL
    assert np.isfinite(got).all()


@pytest.mark.parametrize("m", [1, 32])
def test_config4_70b_shapes(backend, oracle, m):
    """LLaMA-70B-shape matrices (hidden 8192, FFN 28672, 8 KV heads): Wk
    (1024 x 8192 Q4_K), a 384-row slice of W_gate's 8192-wide rows (Q4_K) and
    a 256-row slice of W_down's 28672-wide rows (Q6_K), at decode batch 1 and
    32; row slices keep the CPU reference within seconds while K, the
    dimension the kernels loop over, is full size."""
    g = synth.rng(70)
    for name, t, n, k in (("wk", GGML_Q4_K, 1024, 8192), ("w_gate", GGML_Q4_K, 384, 8192),
                          ("w_down", GGML_Q6_K, 256, 28672)):
        blocks = synth.blocks(g, t, n, k)
        x = synth.activations(g, m, k)
        h = backend.register_weights(t, blocks, n, k)
        try:
            got = backend.weights_matmul(h, x)
        finally:
            backend.release_weights(h)
        rc, ref = oracle.candle_fused(t, blocks, x, m, n, k)
        err = rel_l2(got, ref)
        print(f"70b {name} m={m} rel_l2={err:.3e}")
        assert rc == 0 and err < REL_TOL, name


def _dev_matmul(backend, t, blocks, n, k, x, bf16):
    """Resident weights, device activations (f32 or bf16 bits), one launch."""
    h = backend.register_weights(t, blocks, n, k)
    m = x.shape[0]
    dx = backend.alloc(x.nbytes).upload(x)
    dy = backend.alloc(m * n * 4)
    try:
        backend.matmul_dev(h, dx.ptr, m, dy.ptr, bf16=bf16)
        backend.synchronize()
        return dy.download(np.float32, m * n).reshape(m, n)
    finally:
        backend.release_weights(h)
        dx.close()
        dy.close()


TILED = [("t4111p2", 1), ("t4111p2", 3), ("t4112p2", 1), ("t4112p2", 4), ("t4112p3", 2),
         ("t8112p4", 1), ("t4112s2", 2), ("t4112b2", 1), ("t4112b2", 2), ("t4112b3", 1),
         ("t4112b4", 3), ("t8112b3", 1), ("t8112b4", 2), ("t4114b2", 1), ("t8111b4", 1)]


@pytest.mark.parametrize("tile,ks", TILED)
@pytest.mark.parametrize("t", [GGML_Q4_K, GGML_Q6_K, GGML_Q8_0])
def test_tiled_variants(backend, oracle, monkeypatch, tile, ks, t):
    """Every LDS-tiled kernel variant (forced through the tuning override):
    ragged rows (N = 300) and tokens, six 256-blocks split unevenly over K
    splits, the packed / separate-lo / bf16 activation modes; Q6_K once
    with sub-scales over the full int8 range (the split-scale decode); Q8_0
    with quants over the full int8 range (-128 included)."""
    monkeypatch.setenv("REALM_GEMM_TILE", tile)
    monkeypatch.setenv("REALM_GEMM_KS", str(ks))
    bf16 = tile.endswith(("b2", "b3", "b4"))
    g = synth.rng(zlib.crc32(f"{tile}{ks}{t}".encode()) % 100000)
    n, k = 300, 1536
    blocks = synth.blocks(g, t, n, k)
    if t == GGML_Q6_K and ks > 1:
        blocks["scales"] = g.integers(-128, 128, blocks["scales"].shape, dtype=np.int8)
    if t == GGML_Q8_0:
        blocks["quants"] = g.integers(-128, 128, blocks["quants"].shape, dtype=np.int8)
    for m in (37, 70):
        if bf16:
            xb = synth.activations_bf16(g, m, k)
            got = _dev_matmul(backend, t, blocks, n, k, xb, True)
            x = synth.bf16_bits_to_f32(xb)
        else:
            x = synth.activations(g, m, k)
            got = _dev_matmul(backend, t, blocks, n, k, x, False)
        assert tile in backend.last_kernel() or "reduce" in backend.last_kernel()
        rc, ref = oracle.candle_fused(t, blocks, x, m, n, k)
        err = rel_l2(got, ref.reshape(m, n))
        print(f"{tile} ks={ks} {NAMES[t]} m={m} rel_l2={err:.3e}")
        assert rc == 0 and err < REL_TOL


@pytest.mark.parametrize("t", FORMATS)
@pytest.mark.parametrize("m", [1, 4, 16, 37])
def test_grouped_launch(backend, oracle, t, m):
    """Up to four matrices that share the input in one call (Q/K/V-like,
    ragged row counts): the grouped GEMV at batch 1, per-matrix
    small-batch tiles, and one LDS-tiled launch over all row tiles (Q4_K /
    Q6_K from 16 tokens), each output against the oracle."""
    g = synth.rng(zlib.crc32(f"group{t}{m}".encode()) % 100000)
    k = 1536
    # 300, 128 and 78 rows start on pass boundaries of the GEMV (2 rows per
    # pass at K = 1536), so batches of 1-4 run one grouped launch; the MFMA
    # paths see ragged row tiles
    ns = (300, 128, 78)
    blocks = [synth.blocks(g, t, n, k) for n in ns]
    x = synth.activations(g, m, k)
    hs = [backend.register_weights(t, b, n, k) for b, n in zip(blocks, ns)]
    dx = backend.alloc(x.nbytes).upload(x)
    dys = [backend.alloc(m * n * 4) for n in ns]
    try:
        outs = []
        for rep in range(2):
            backend.matmul_group_dev(hs, dx.ptr, m, [d.ptr for d in dys])
            backend.synchronize()
            outs.append([d.download(np.float32, m * n).reshape(m, n) for d, n in zip(dys, ns)])
        kernel = backend.last_kernel()
    finally:
        for h in hs:
            backend.release_weights(h)
        dx.close()
        for d in dys:
            d.close()
    if m >= 16 and t != GGML_Q8_0:
        assert "_t41" in kernel or "tiled_reduce" in kernel, kernel
    if m <= 4:  # one grouped GEMV launch for all three matrices
        assert kernel.startswith("realm_gemv_") and "_m4" in kernel, kernel
    for i, (b, n) in enumerate(zip(blocks, ns)):
        assert bits_equal(outs[0][i], outs[1][i])  # repeatable
        rc, ref = oracle.candle_fused(t, b, x, m, n, k)
        err = rel_l2(outs[0][i], ref.reshape(m, n))
        print(f"group {NAMES[t]} m={m} mat {i} n={n} rel_l2={err:.3e}")
        assert rc == 0 and err < REL_TOL


def test_grouped_q6k_mixed_wide(backend, oracle):
    """A grouped Q6_K launch where one matrix has sub-scales over the full
    int8 range (the split-scale decode) and the others do not: the whole
    launch takes the wide decode, exact for both kinds."""
    g = synth.rng(606)
    k, m = 1536, 37
    ns = (200, 96, 130)
    blocks = [synth.blocks(g, GGML_Q6_K, n, k) for n in ns]
    blocks[1]["scales"] = g.integers(-128, 128, blocks[1]["scales"].shape, dtype=np.int8)
    x = synth.activations(g, m, k)
    hs = [backend.register_weights(GGML_Q6_K, b, n, k) for b, n in zip(blocks, ns)]
    dx = backend.alloc(x.nbytes).upload(x)
    dys = [backend.alloc(m * n * 4) for n in ns]
    try:
        backend.matmul_group_dev(hs, dx.ptr, m, [d.ptr for d in dys])
        backend.synchronize()
        kernel = backend.last_kernel()
        got = [d.download(np.float32, m * n).reshape(m, n) for d, n in zip(dys, ns)]
    finally:
        for h in hs:
            backend.release_weights(h)
        for d in [dx] + dys:
            d.close()
    assert "q6kw_t" in kernel or "tiled_reduce" in kernel, kernel
    for b, n, gi in zip(blocks, ns, got):
        rc, ref = oracle.candle_fused(GGML_Q6_K, b, x, m, n, k)
        assert rc == 0 and rel_l2(gi, ref.reshape(m, n)) < REL_TOL


@pytest.mark.parametrize("t", FORMATS)
@pytest.mark.parametrize("m", [2, 3, 4])
def test_gemv_tokens(backend, oracle, t, m):
    """The multi-token integer-dot GEMV (2 tokens; 3 and 4 on the 4-token
    kernels): every lanes-per-row / units-per-lane shape from K = 1024 to
    28672, ragged row counts, one matrix and a grouped launch.  Each output
    is checked against the oracle, and each token's row against a one-token
    launch on that token alone (the same quantized x and the same integer
    sums, so they agree to f32 rounding)."""
    g = synth.rng(zlib.crc32(f"tokens{t}{m}".encode()) % 100000)
    suffix = "_t2" if m == 2 else "_t4"
    for n, k in ((37, 1024), (50, 2048), (45, 4096), (33, 11008), (19, 28672)):
        blocks = synth.blocks(g, t, n, k)
        x = synth.activations(g, m, k)
        got = _dev_matmul(backend, t, blocks, n, k, x, False)
        kernel = backend.last_kernel()
        # 4 tokens of a 28672-long row need more LDS than a workgroup has:
        # those go to the MFMA path
        if not (k == 28672 and m > 2):
            assert kernel.startswith("realm_gemv_") and kernel.endswith(suffix), kernel
        rc, ref = oracle.candle_fused(t, blocks, x, m, n, k)
        err = rel_l2(got, ref.reshape(m, n))
        print(f"{NAMES[t]} m={m} n={n} k={k} {kernel} rel_l2={err:.3e}")
        assert rc == 0 and err < REL_TOL, (n, k)
        if kernel.startswith("realm_gemv_"):
            for i in range(m):
                one = _dev_matmul(backend, t, blocks, n, k, x[i:i + 1], False)
                assert np.max(np.abs(one[0] - got[i])) <= 1e-6 * np.max(np.abs(one[0])), (k, i)
    # grouped: three matrices of one row each per pass (K = 4096)
    k, ns = 4096, (64, 40, 24)
    blocks = [synth.blocks(g, t, n, k) for n in ns]
    x = synth.activations(g, m, k)
    hs = [backend.register_weights(t, b, n, k) for b, n in zip(blocks, ns)]
    dx = backend.alloc(x.nbytes).upload(x)
    dys = [backend.alloc(m * n * 4) for n in ns]
    try:
        backend.matmul_group_dev(hs, dx.ptr, m, [d.ptr for d in dys])
        backend.synchronize()
        kernel = backend.last_kernel()
        outs = [d.download(np.float32, m * n).reshape(m, n) for d, n in zip(dys, ns)]
    finally:
        for h in hs:
            backend.release_weights(h)
        dx.close()
        for d in dys:
            d.close()
    assert "_m4" + suffix in kernel, kernel
    for b, n, got in zip(blocks, ns, outs):
        rc, ref = oracle.candle_fused(t, b, x, m, n, k)
        assert rc == 0 and rel_l2(got, ref.reshape(m, n)) < REL_TOL, n


@pytest.mark.parametrize("ks", [2, 3, 6])
def test_tiled_ksplit_repeat(backend, oracle, monkeypatch, ks):
    """K-split parts summed in split order: results are bit-identical from
    call to call, also when calls of different shapes (and part-buffer
    sizes) alternate on one stream."""
    monkeypatch.setenv("REALM_GEMM_TILE", "t4112p2")
    monkeypatch.setenv("REALM_GEMM_KS", str(ks))
    g = synth.rng(500 + ks)
    k = 1536
    cases = [(GGML_Q4_K, 300, 37), (GGML_Q6_K, 520, 70), (GGML_Q4_K, 129, 16)]
    data = [(t, n, m, synth.blocks(g, t, n, k), synth.activations(g, m, k)) for t, n, m in cases]
    first = {}
    for rep in range(3):
        for i, (t, n, m, b, x) in enumerate(data):
            got = _dev_matmul(backend, t, b, n, k, x, False)
            if rep == 0:
                first[i] = got
                rc, ref = oracle.candle_fused(t, b, x, m, n, k)
                assert rc == 0 and rel_l2(got, ref.reshape(m, n)) < REL_TOL
            else:
                assert bits_equal(got, first[i]), (rep, i)


def test_q6k_wide_scales(backend, oracle):
    """Q6_K sub-scales over the full int8 range use the split-scale path."""
    g = synth.rng(66)
    n, k = 96, 2048
    blocks = synth.q6k_blocks(g, n, k)
    blocks["scales"] = g.integers(-128, 128, blocks["scales"].shape, dtype=np.int8)
    for m in (1, 8, 40):
        x = synth.activations(g, m, k)
        got = backend.fused_dequant_matmul_q6k(blocks, x, m, n, k)
        rc, ref = oracle.candle_fused(GGML_Q6_K, blocks, x, m, n, k)
        assert rc == 0 and rel_l2(got, ref) < REL_TOL, m


@pytest.mark.parametrize("scale", [1e-30, 1e-6, 1e6, 1e30])
def test_activation_range(backend, oracle, scale):
    """Activations far outside f16 range stay exact through the per-token
    power-of-two rescale of the MFMA path (and the f32 GEMV path)."""
    g = synth.rng(55)
    n, k = 64, 1024
    blocks = synth.q4k_blocks(g, n, k)
    for m in (1, 20):
        x = synth.activations(g, m, k) * np.float32(scale)
        x[:, 5] *= 1e3  # a large outlier per token
        got = backend.fused_dequant_matmul_q4k(blocks, x, m, n, k)
        rc, ref = oracle.candle_fused(GGML_Q4_K, blocks, x, m, n, k)
        assert rc == 0 and rel_l2(got, ref) < REL_TOL, (scale, m)


def test_nan_fallback(backend, oracle):
    g = synth.rng(8)
    n, k = 32, 512
    blocks = synth.q4k_blocks(g, n, k)
    blocks["d"][::7] = 0x7E00
    for m in (1, 24):
        x = synth.activations(g, m, k)
        got = backend.fused_dequant_matmul_q4k(blocks, x, m, n, k)
        rc, ref = oracle.candle_fused(GGML_Q4_K, blocks, x, m, n, k)
        assert np.array_equal(np.isnan(got), np.isnan(ref))
        backend.set_nan_fallback(True)
        try:
            got = backend.fused_dequant_matmul_q4k(blocks, x, m, n, k)
        finally:
            backend.set_nan_fallback(False)
        rc, ref = oracle.fused(GGML_Q4_K, blocks, x, m, n, k, nan_fallback=True)
        assert np.isfinite(got).all() and rel_l2(got, ref) < REL_TOL


# ------------------------------------------------------------------- LoRA

def _oracle_lora(oracle, t, blocks, x, ids, adapters, n, k):
    m = x.shape[0]
    rc, base = oracle.candle_fused(t, blocks, x, m, n, k)
    assert rc == 0
    ad = [(a.astype(np.float32), b.astype(np.float32), r, al) for a, b, r, al in adapters]
    return oracle.multi_lora_delta(x, ids, ad, base.reshape(m, n).copy())


@pytest.mark.parametrize("t", FORMATS)
@pytest.mark.parametrize("dtype", [np.float16, np.float32])
@pytest.mark.parametrize("shape", [(160, 512, 37), (600, 1536, 70)])
def test_multi_lora_small(backend, oracle, t, dtype, shape):
    """Ranks 3 (not a multiple of 8) to 100 (past the 64 the expand holds in
    registers); the second shape has several row groups and K parts."""
    g = synth.rng(300 + t + shape[0])
    n, k, m = shape
    blocks = synth.blocks(g, t, n, k)
    x = synth.activations(g, m, k)
    adapters, handles = [], []
    for r in (8, 16, 64, 3, 100):
        a, b = synth.lora_adapter(g, r, k, n)
        a, b = a.astype(dtype), b.astype(dtype)
        adapters.append((a, b, r, 16.0))
        handles.append(backend.lora_register(a, b, r, 16.0, k, n))
    ids = synth.adapter_ids(g, m, len(adapters))
    ids[3] = 99  # unknown slot: base only
    wh = backend.register_weights(t, blocks, n, k)
    sh = backend.lora_set_create(handles)
    try:
        got = backend.multi_lora_matmul(wh, sh, x, ids)
        base = backend.weights_matmul(wh, x)
    finally:
        backend.lora_set_release(sh)
        for h in handles:
            backend.lora_release(h)
        backend.release_weights(wh)
    ref = _oracle_lora(oracle, t, blocks, x, ids, adapters, n, k)
    assert rel_l2(got, ref) < REL_TOL
    none = (ids < 0) | (ids >= len(adapters))
    assert np.array_equal(got[none], base[none]) or rel_l2(got[none], base[none]) < 1e-6


@pytest.mark.parametrize("scale", [1e-30, 1e-6, 1e6, 1e20, 1e30])
@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_multi_lora_activation_range(backend, oracle, scale, dtype):
    """u = A x takes the activations' units: at 1e6 and beyond it is far past
    f16 range (the expand rescales it per token by a power of two before its
    f16 split); at 1e-30 and 1e30 (with a 1e3 outlier: max |x| outside
    [2^-60, 2^100]) the tokens take the exact f32 path, and their u comes from
    the caller's activations in f32 — the LoRA delta is kept, as the
    reference's y = W x + s B (A x) (lora.rs:91-144) keeps it for any finite
    x.  Single products and a grouped one, 1, 6 and 40 tokens."""
    g = synth.rng(77)
    n, k = 192, 1024
    blocks = synth.q4k_blocks(g, n, k)
    adapters, handles = [], []
    for r in (8, 19):
        a, b = synth.lora_adapter(g, r, k, n)
        a, b = a.astype(dtype), (b.astype(np.float32) * 20).astype(dtype)
        adapters.append((a, b, r, 16.0))
        handles.append(backend.lora_register(a, b, r, 16.0, k, n))
    wh = backend.register_weights(GGML_Q4_K, blocks, n, k)
    sh = backend.lora_set_create(handles)
    try:
        for m in (1, 6, 40):
            x = synth.activations(g, m, k) * np.float32(scale)
            x[:, 5] *= 1e3  # a large outlier per token
            ids = (np.arange(m) % 3).astype(np.int32)  # slot 2: no adapter
            ref = _oracle_lora(oracle, GGML_Q4_K, blocks, x, ids, adapters, n, k)
            base = _oracle_lora(oracle, GGML_Q4_K, blocks, x, np.full(m, -1, np.int32),
                                adapters, n, k)
            assert np.isfinite(ref).all() and rel_l2(ref, base) > 1e-2  # deltas matter
            got = backend.multi_lora_matmul(wh, sh, x, ids)
            assert np.isfinite(got).all() and rel_l2(got, ref) < REL_TOL, (scale, m)
            dx = backend.alloc(x.nbytes).upload(x)
            d_ids = backend.alloc(ids.nbytes).upload(ids)
            dys = [backend.alloc(m * n * 4) for _ in range(2)]
            try:
                backend.multi_lora_matmul_group_dev([wh, wh], [sh, sh], dx.ptr, m, d_ids.ptr,
                                                    [d.ptr for d in dys])
                backend.synchronize()
                for d in dys:
                    gy = d.download(np.float32, m * n).reshape(m, n)
                    assert rel_l2(gy, ref) < REL_TOL, ("group", scale, m)
            finally:
                for b_ in [dx, d_ids] + dys:
                    b_.close()
    finally:
        backend.lora_set_release(sh)
        for h in handles:
            backend.lora_release(h)
        backend.release_weights(wh)


@pytest.mark.parametrize("t", [GGML_Q4_K, GGML_Q6_K, GGML_Q8_0])
@pytest.mark.parametrize("m", [4, 37])
@pytest.mark.parametrize("rt", ["fused", "", "2", "4", "8"])
def test_multi_lora_group(backend, oracle, monkeypatch, t, m, rt):
    """q/k/v-like projections with their own adapter sets in one grouped
    call (ragged rows; ranks 3 to 100; f16 and f32 factors), against the
    oracle per projection: per-matrix launches at 4 tokens, one tiled base
    launch for the group at 37.  At 37 tokens, "fused" (the default): the
    shrink runs in the xprep launch and the expand in the K-split reduce
    (the last kernel); otherwise (REALM_LORA_FUSED=0) one shrink and one
    expand launch for the group, the expand with its default row tile and
    each of 128, 256 and 512 rows per workgroup forced (600 rows: several
    row groups, the last one partial; shorter projections skip the groups
    past their rows)."""
    if rt != "fused":
        monkeypatch.setenv("REALM_LORA_FUSED", "0")
    if rt not in ("fused", ""):
        monkeypatch.setenv("REALM_LORA_EXPAND_RT", rt)
    g = synth.rng(zlib.crc32(f"lgroup{t}{m}".encode()) % 100000)
    k = 1536
    specs = [(600, (8, 16, 3), np.float16), (128, (64,), np.float32), (77, (100, 8), np.float16)]
    x = synth.activations(g, m, k)
    ids = synth.adapter_ids(g, m, 3)
    ids[1] = 7  # unknown slot where a projection has fewer adapters: base only
    whs, shs, lhs, refs, ns = [], [], [], [], []
    dx = backend.alloc(x.nbytes).upload(x)
    d_ids = backend.alloc(ids.nbytes).upload(ids)
    dys = []
    try:
        for n, ranks, dt in specs:
            blocks = synth.blocks(g, t, n, k)
            adapters, hs = [], []
            for r in ranks:
                a, b = synth.lora_adapter(g, r, k, n)
                a, b = a.astype(dt), b.astype(dt)
                adapters.append((a, b, r, 16.0))
                hs.append(backend.lora_register(a, b, r, 16.0, k, n))
            lhs += hs
            whs.append(backend.register_weights(t, blocks, n, k))
            shs.append(backend.lora_set_create(hs))
            refs.append(_oracle_lora(oracle, t, blocks, x, ids, adapters, n, k))
            ns.append(n)
            dys.append(backend.alloc(m * n * 4))
        backend.multi_lora_matmul_group_dev(whs, shs, dx.ptr, m, d_ids.ptr, [d.ptr for d in dys])
        backend.synchronize()
        kernel = backend.last_kernel()
        got = [d.download(np.float32, m * n).reshape(m, n) for d, n in zip(dys, ns)]
    finally:
        for sh in shs:
            backend.lora_set_release(sh)
        for h in lhs:
            backend.lora_release(h)
        for wh in whs:
            backend.release_weights(wh)
        for d in [dx, d_ids] + dys:
            d.close()
    if m > 4 and rt == "fused":  # the expand is in the reduce
        assert kernel == "realm_gemm_tiled_reduce_lora", kernel
    elif m > 4:  # one expand launch for the group is the last kernel
        assert kernel.startswith("realm_lora_expand"), kernel
        if rt:
            assert kernel.endswith("expand" if rt == "8" else f"_rt{rt}"), kernel
    for i, (gi, ref) in enumerate(zip(got, refs)):
        err = rel_l2(gi, ref)
        print(f"lora group {NAMES[t]} m={m} rt={rt} proj {i} rel_l2={err:.3e}")
        assert err < REL_TOL


def test_multi_lora_config3(backend, oracle):
    """16 tenants, ranks from {8,16,64}, 64 tokens with Zipf(1.1) ids and 10%
    no-adapter, on a shared Q4_K 4096 x 4096 projection."""
    g = synth.rng(3)
    n = k = 4096
    m = 64
    blocks = synth.q4k_blocks(g, n, k)
    ranks = g.choice([8, 16, 64], 16)
    adapters = []
    for r in ranks:
        a, b = synth.lora_adapter(g, int(r), k, n)
        adapters.append((a, b, int(r), 16.0))
    ids = synth.adapter_ids(g, m, 16)
    x = synth.activations(g, m, k)
    handles = [backend.lora_register(a, b, r, al, k, n) for a, b, r, al in adapters]
    wh = backend.register_weights(GGML_Q4_K, blocks, n, k)
    sh = backend.lora_set_create(handles)
    try:
        got = backend.multi_lora_matmul(wh, sh, x, ids)
    finally:
        backend.lora_set_release(sh)
        for h in handles:
            backend.lora_release(h)
        backend.release_weights(wh)
    ref = _oracle_lora(oracle, GGML_Q4_K, blocks, x, ids, adapters, n, k)
    err = rel_l2(got, ref)
    # the LoRA delta itself, not just the sum, must match
    rc, base = oracle.candle_fused(GGML_Q4_K, blocks, x, m, n, k)
    derr = rel_l2(got - base.reshape(m, n), ref - base.reshape(m, n))
    print(f"config3 rel_l2={err:.3e} delta rel_l2={derr:.3e}")
    assert err < REL_TOL and derr < 1e-2


def test_lora_validation(backend):
    a = np.zeros((4, 256), np.float16)
    b = np.zeros((64, 4), np.float16)
    with pytest.raises(InvalidShape):
        backend.lora_register(a, b, 0, 1.0, 256, 64)
    h = backend.lora_register(a, b, 4, 8.0, 256, 64)
    sh = backend.lora_set_create([h])
    with pytest.raises(InvalidShape):  # in use by a set
        backend.lora_release(h)
    wh = backend.register_weights(GGML_Q4_K, synth.q4k_blocks(synth.rng(1), 32, 256), 32, 256)
    with pytest.raises(InvalidShape):  # dims differ from the weight
        backend.multi_lora_matmul(wh, sh, np.zeros((1, 256), np.float32), np.zeros(1, np.int32))
    backend.release_weights(wh)
    backend.lora_set_release(sh)
    backend.lora_release(h)


# ------------------------------------------------------------------ dense

def test_dense_kats(backend, kat):
    assert np.array_equal(backend.matmul(kat["dense_a1"], kat["dense_b1"], 2, 3, 2),
                          kat["dense_e1"])
    assert np.array_equal(backend.matmul(kat["dense_a3"], kat["dense_b3"], 2, 2, 2),
                          kat["dense_e3"])
    with pytest.raises(RealmError):
        backend.matmul(kat["dense_a1"], kat["dense_b1"], 2, 2, 2)


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (3, 5, 7), (64, 64, 64), (65, 130, 33),
                                   (200, 300, 100)])
def test_dense_random(backend, m, k, n):
    g = synth.rng(m * 7 + k)
    a = g.standard_normal((m, k), dtype=np.float32)
    b = g.standard_normal((k, n), dtype=np.float32)
    got = backend.matmul(a, b, m, k, n).reshape(m, n)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert rel_l2(got, ref) < 1e-5


@pytest.mark.parametrize("transposed", [False, True])
@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (2, 3, 2), (31, 17, 129), (128, 256, 128),
                                   (130, 515, 257), (32, 2048, 300), (5, 4099, 70),
                                   (33, 1024, 200), (64, 700, 130), (65, 300, 129)])
def test_dense_dev(backend, m, k, n, transposed):
    """Device-pointer dense product, both B layouts, ragged tile edges in m,
    n and k, skinny products with K splits (parts summed in split order) on
    the 32- and 64-row tiles: f32 products and sums, so within f32 rounding
    of an f64 product; small-integer inputs give exact results."""
    g = synth.rng(m * 131 + k * 7 + n + transposed)
    for ints in (False, True):
        if ints:
            a = g.integers(-8, 9, (m, k)).astype(np.float32)
            b = g.integers(-8, 9, (k, n)).astype(np.float32)
        else:
            a = g.standard_normal((m, k), dtype=np.float32)
            b = g.standard_normal((k, n), dtype=np.float32)
        bs = np.ascontiguousarray(b.T) if transposed else b
        da, db = backend.alloc(a.nbytes).upload(a), backend.alloc(bs.nbytes).upload(bs)
        dc = backend.alloc(m * n * 4)
        try:
            backend.dense_matmul_dev(da.ptr, db.ptr, dc.ptr, m, k, n, transposed=transposed)
            backend.synchronize()
            got = dc.download(np.float32, m * n).reshape(m, n)
        finally:
            for d in (da, db, dc):
                d.close()
        ref = a.astype(np.float64) @ b.astype(np.float64)
        if ints:
            assert np.array_equal(got, ref.astype(np.float32))
        else:  # f32 sums over k: relative error about 2^-24 sqrt(k)
            assert rel_l2(got, ref) < 1e-5
    tile = "realm_dense_f32" + ("_m32" if m <= 32 else "_m64" if m <= 64 else "")
    assert backend.last_kernel() in (tile, "realm_dense_reduce"), backend.last_kernel()


def test_candle_matmul_host_function(backend, kat):
    """env.candle_matmul over a linear memory (memory64_host.rs:853-1086)."""
    mem = np.zeros(4096, np.uint8)
    a, b = kat["dense_a2"], kat["dense_bt2"]
    mem[100:116] = a.view(np.uint8)  # unaligned offsets are allowed
    mem[203:219] = b.view(np.uint8)
    rc = backend.candle_matmul(mem, 100, 203, 301, 2, 2, 2, transposed=True)
    assert rc == 4
    assert np.array_equal(mem[301:317].copy().view(np.float32), kat["dense_e2"])
    mem[203:219] = np.array([1, 2, 3, 4], np.float32).view(np.uint8)
    rc = backend.candle_matmul(mem, 100, 203, 301, 2, 2, 2)
    assert rc == 4 and np.array_equal(mem[301:317].copy().view(np.float32),
                                      np.array([7, 10, 15, 22], np.float32))
    assert backend.candle_matmul(mem, 4090, 0, 0, 2, 2, 2) == -3
    assert backend.candle_matmul(mem, 0, 4090, 0, 2, 2, 2) == -4
    assert backend.candle_matmul(mem, 0, 0, 4090, 2, 2, 2) == -6


# ------------------------------------------------------- device-pointer path

def test_resident_dev_path_and_events(backend, oracle):
    g = synth.rng(12)
    n, k, m = 512, 2048, 8
    blocks = synth.q4k_blocks(g, n, k)
    x = synth.activations(g, m, k)
    h = backend.register_weights(GGML_Q4_K, blocks, n, k)
    assert backend.weights_info(h)[:3] == (GGML_Q4_K, n, k)
    dx = backend.alloc(x.nbytes).upload(x)
    dy = backend.alloc(m * n * 4)
    s = backend.stream()
    e0, e1 = backend.event(), backend.event()
    try:
        backend.record(e0, s)
        backend.matmul_dev(h, dx.ptr, m, dy.ptr, stream=s)
        backend.record(e1, s)
        assert backend.elapsed_ms(e0, e1) >= 0.0
        got = dy.download(np.float32, m * n)
        # repeated calls give identical results
        backend.matmul_dev(h, dx.ptr, m, dy.ptr, stream=s)
        backend.synchronize()
        assert np.array_equal(dy.download(np.float32, m * n), got)
    finally:
        backend.release_weights(h)
        dx.close()
        dy.close()
    rc, ref = oracle.candle_fused(GGML_Q4_K, blocks, x, m, n, k)
    assert rel_l2(got, ref) < REL_TOL
    with pytest.raises(InvalidShape):
        backend.weights_matmul(h, x)  # released handle

"""GPU parity at exactly the shapes and kernels bench.py times, and at the
config-4 (LLaMA-70B layer) prefill and multi-LoRA shapes.

Each product runs through the C ABI and is checked against the CPU oracle
(CandleCpuBackend semantics: dequantize, then f32 x . W^T) within 1e-3
relative L2 (REL_TOL); large matrices are checked on a seeded subset of
output rows, with K, the dimension the kernels loop over, at full size.
The kernel each launch ran is asserted, so the timed variants cannot drift
away from the tested ones.
"""
import numpy as np
import pytest

from realm_amd import synth
from realm_amd.formats import GGML_Q4_K, GGML_Q6_K

from conftest import rel_l2

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3


def _rows(t, blocks, n, k, rows):
    return blocks.reshape(n, k // 256)[rows].reshape(-1)


def _check(oracle, t, blocks, x, got, n, k, rows=None, tag=""):
    m = x.shape[0]
    if rows is None:
        rc, ref = oracle.candle_fused(t, blocks, x, m, n, k)
        g = got
    else:
        rc, ref = oracle.candle_fused(t, _rows(t, blocks, n, k, rows), x, m, rows.size, k)
        g = got[:, rows]
    assert rc == 0
    err = rel_l2(g, ref.reshape(m, -1))
    print(f"{tag} rel_l2={err:.3e}")
    assert err < REL_TOL, tag


# The bench's decode step: per layer Q/K/V grouped, Wo, gate/up grouped,
# W_down, batch 1, LLaMA-7B shapes; the kernel names are the variants the
# host picks on a 256-CU MI355X (the roofline kernel is the gate/up one).
BENCH_LAUNCHES = [
    ("qkv", GGML_Q4_K, (4096, 4096, 4096), 4096, "realm_gemv_q4k_l64_u1_d1_m4"),
    ("wo", GGML_Q4_K, (4096,), 4096, "realm_gemv_q4k_l64_u1_d1_m1"),
    ("gate_up", GGML_Q4_K, (11008, 11008), 4096, "realm_gemv_q4k_l64_u1_d2_m4"),
    ("w_down", GGML_Q6_K, (4096,), 11008, "realm_gemv_q6k_l64_u3_d2_m1"),
]


@pytest.mark.parametrize("name,t,ns,k,kernel", BENCH_LAUNCHES,
                         ids=[b[0] for b in BENCH_LAUNCHES])
def test_bench_decode_launch(backend, oracle, name, t, ns, k, kernel):
    g = synth.rng(7000 + len(name))
    blocks = [synth.blocks(g, t, n, k) for n in ns]
    x = synth.activations(g, 1, k)
    hs = [backend.register_weights(t, b, n, k) for b, n in zip(blocks, ns)]
    dx = backend.alloc(x.nbytes).upload(x)
    dys = [backend.alloc(4 * n) for n in ns]
    try:
        if len(hs) == 1:
            backend.matmul_dev(hs[0], dx.ptr, 1, dys[0].ptr)
        else:
            backend.matmul_group_dev(hs, dx.ptr, 1, [d.ptr for d in dys])
        backend.synchronize()
        ran = backend.last_kernel()
        outs = [d.download(np.float32, n).reshape(1, n) for d, n in zip(dys, ns)]
    finally:
        for h in hs:
            backend.release_weights(h)
        for d in [dx] + dys:
            d.close()
    assert ran == kernel, ran
    for i, (b, n, y) in enumerate(zip(blocks, ns, outs)):
        _check(oracle, t, b, x, y, n, k, tag=f"{name}[{i}] {ran}")


@pytest.mark.parametrize("depth", [1, 2, 3, 4, 6, 8, 12])
def test_gemv_ring_depths_grouped(backend, oracle, monkeypatch, depth):
    """Every ring depth of the one-unit-per-lane GEMV forced on a grouped
    launch of four 4096-wide Q4_K matrices (one of them ragged against the
    passes of the deeper rings)."""
    monkeypatch.setenv("REALM_GEMV_D", str(depth))
    g = synth.rng(7100 + depth)
    k, ns = 4096, (3072, 1024, 2048, 1000)
    blocks = [synth.blocks(g, GGML_Q4_K, n, k) for n in ns]
    x = synth.activations(g, 1, k)
    hs = [backend.register_weights(GGML_Q4_K, b, n, k) for b, n in zip(blocks, ns)]
    dx = backend.alloc(x.nbytes).upload(x)
    dys = [backend.alloc(4 * n) for n in ns]
    try:
        backend.matmul_group_dev(hs, dx.ptr, 1, [d.ptr for d in dys])
        backend.synchronize()
        ran = backend.last_kernel()
        outs = [d.download(np.float32, n).reshape(1, n) for d, n in zip(dys, ns)]
    finally:
        for h in hs:
            backend.release_weights(h)
        for d in [dx] + dys:
            d.close()
    assert ran == f"realm_gemv_q4k_l64_u1_d{depth}_m4", ran
    for i, (b, n, y) in enumerate(zip(blocks, ns, outs)):
        _check(oracle, GGML_Q4_K, b, x, y, n, k, tag=f"d{depth}[{i}]")


# ----------------------------------------------------------- config 4

@pytest.mark.parametrize("name,t,n,k,kernel", [
    ("w_gate", GGML_Q4_K, 28672, 8192, "realm_gemm_q4k_t4112b2"),
    ("w_down", GGML_Q6_K, 8192, 28672, "realm_gemm_q6k_t4112b2"),
])
def test_config4_prefill_1024(backend, oracle, name, t, n, k, kernel):
    """The config-4 1024-token bf16 prefill on the full 70B-shape W_gate
    (Q4_K, K = 8192) and W_down (Q6_K, K = 28672), the launches bench.py
    times; checked on 48 seeded rows for all 1024 tokens."""
    g = synth.rng(7400 + k)
    m = 1024
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
    assert ran == kernel or ran == "realm_gemm_tiled_reduce", ran
    rows = np.sort(synth.rng(7401).choice(n, 48, replace=False))
    _check(oracle, t, blocks, synth.bf16_bits_to_f32(xb), got, n, k, rows=rows,
           tag=f"config4 prefill {name} {ran}")
    assert np.isfinite(got).all()


def test_config4_lora_qkvo(backend, oracle):
    """Config 4's decode: 32 tokens, 8 rank-16 adapters on each of q, k, v
    (one grouped multi-LoRA call, K = 8192, GQA k/v 1024 rows) and o (a
    single call), as bench.py runs it; base and LoRA delta checked per
    projection on seeded row subsets (the adapters' B rows sliced with
    them)."""
    g = synth.rng(7500)
    m, k = 32, 8192
    specs = [("q", 8192), ("k", 1024), ("v", 1024), ("o", 8192)]
    x = synth.activations(g, m, k)
    ids = synth.adapter_ids(g, m, 8)
    dx = backend.alloc(x.nbytes).upload(x)
    d_ids = backend.alloc(ids.nbytes).upload(ids)
    whs, shs, lhs, dys, host = [], [], [], [], []
    try:
        for name, n in specs:
            blocks = synth.blocks(g, GGML_Q4_K, n, k)
            adapters, hs = [], []
            for _ in range(8):
                a, b = synth.lora_adapter(g, 16, k, n)
                adapters.append((a, b, 16, 16.0))
                hs.append(backend.lora_register(a, b, 16, 16.0, k, n))
            lhs += hs
            whs.append(backend.register_weights(GGML_Q4_K, blocks, n, k))
            shs.append(backend.lora_set_create(hs))
            dys.append(backend.alloc(m * n * 4))
            host.append((name, n, blocks, adapters))
        backend.multi_lora_matmul_group_dev(whs[:3], shs[:3], dx.ptr, m, d_ids.ptr,
                                            [d.ptr for d in dys[:3]])
        backend.multi_lora_matmul_dev(whs[3], shs[3], dx.ptr, m, d_ids.ptr, dys[3].ptr)
        backend.synchronize()
        got = [d.download(np.float32, m * n).reshape(m, n) for d, (_, n) in zip(dys, specs)]
    finally:
        for sh in shs:
            backend.lora_set_release(sh)
        for h in lhs:
            backend.lora_release(h)
        for wh in whs:
            backend.release_weights(wh)
        for d in [dx, d_ids] + dys:
            d.close()
    for (name, n, blocks, adapters), y in zip(host, got):
        rows = np.sort(synth.rng(7501 + n).choice(n, min(n, 192), replace=False))
        rc, base = oracle.candle_fused(GGML_Q4_K, _rows(GGML_Q4_K, blocks, n, k, rows), x, m,
                                       rows.size, k)
        assert rc == 0
        ad = [(a.astype(np.float32), b.astype(np.float32)[rows], r, al)
              for a, b, r, al in adapters]
        base = base.reshape(m, rows.size)
        ref = oracle.multi_lora_delta(x, ids, ad, base.copy())
        err = rel_l2(y[:, rows], ref)
        derr = rel_l2(y[:, rows] - base, ref - base)
        print(f"config4 lora {name} rel_l2={err:.3e} delta rel_l2={derr:.3e}")
        assert err < REL_TOL and derr < 1e-2, name


def test_checksum(backend):
    """realm_hip_checksum: XOR of the little-endian words of a device
    buffer, a trailing partial word zero-padded (numpy restatement), for
    sizes around the 16-byte chunking, and through the _dev form's
    partials."""
    g = np.random.default_rng(77)
    for nbytes in (1, 15, 16, 17, 4096, 1_000_003, 50_000_000):
        host = g.integers(0, 256, nbytes, dtype=np.uint8)
        padded = np.zeros((nbytes + 3) // 4 * 4, np.uint8)
        padded[:nbytes] = host
        want = int(np.bitwise_xor.reduce(padded.view("<u4"))) if padded.size else 0
        d = backend.alloc(nbytes).upload(host)
        try:
            assert backend.checksum(d) == want, nbytes
            parts = backend.alloc(256 * 4)
            backend.checksum_dev(d.ptr, nbytes, parts.ptr, 256)
            backend.synchronize()
            got = int(np.bitwise_xor.reduce(parts.download(np.uint32, 256)))
            parts.close()
            assert got == want, nbytes
        finally:
            d.close()


# ---------------------------------------- graphs and scratch buffers

def test_graph_survives_workspace_growth(backend, oracle):
    """A graph captured on a stream keeps using the scratch buffers it was
    captured with: a later, larger eager call on that stream gets new ones
    and the old ones are kept (not freed) until the graph is released, so
    the replay after the growth still writes the right result.  Runs on a
    thread of its own: the library's stream (and scratch) is per thread, so
    earlier tests on this thread may have grown the buffers already."""
    import threading
    err = []

    def body():
        try:
            _graph_survives_workspace_growth(backend, oracle)
        except BaseException as e:  # re-raised on the test's thread
            err.append(e)
    th = threading.Thread(target=body)
    th.start()
    th.join()
    if err:
        raise err[0]


def _graph_survives_workspace_growth(backend, oracle):
    g = synth.rng(7600)
    n, k = 512, 2048
    blocks = synth.blocks(g, GGML_Q4_K, n, k)
    x_small = synth.activations(g, 16, k)
    x_big = synth.activations(g, 256, k)
    h = backend.register_weights(GGML_Q4_K, blocks, n, k)
    s = backend.stream()
    dxs = backend.alloc(x_small.nbytes).upload(x_small)
    dxb = backend.alloc(x_big.nbytes).upload(x_big)
    dys = backend.alloc(16 * n * 4)
    dyb = backend.alloc(256 * n * 4)
    try:
        backend.matmul_dev(h, dxs.ptr, 16, dys.ptr, stream=s)  # sizes the buffers
        backend.synchronize()
        want = dys.download(np.float32, 16 * n)
        backend.graph_begin(s)
        backend.matmul_dev(h, dxs.ptr, 16, dys.ptr, stream=s)
        gr = backend.graph_end(s)
        _, retired0, graphs = backend.workspace_info(s)
        assert graphs >= 1
        backend.matmul_dev(h, dxb.ptr, 256, dyb.ptr, stream=s)  # grows the buffers
        backend.synchronize()
        _, retired1, _ = backend.workspace_info(s)
        assert retired1 > retired0  # the graph's buffers were kept, not freed
        for _ in range(3):
            dys.upload(np.zeros(16 * n, np.float32))
            backend.graph_launch(gr, s)
            backend.synchronize()
            assert np.array_equal(dys.download(np.float32, 16 * n), want)
        backend.graph_release(gr)
        _, retired2, graphs2 = backend.workspace_info(s)
        assert graphs2 == graphs - 1
        if graphs2 == 0:  # the stream's last graph: the kept buffers are freed
            assert retired2 == 0
        big = dyb.download(np.float32, 256 * n).reshape(256, n)
    finally:
        backend.release_weights(h)
        for d in (dxs, dxb, dys, dyb):
            d.close()
    _check(oracle, GGML_Q4_K, blocks, x_big, big, n, k, tag="after growth")


def test_dense_k0_in_graph(backend):
    """A dense product with k = 0 zero-fills C with a kernel (no memset node
    in a captured graph); replays refill what the eager work overwrote."""
    m, n = 3, 70
    s = backend.stream()
    dc = backend.alloc(m * n * 4)
    dummy = backend.alloc(256)
    try:
        backend.graph_begin(s)
        backend.dense_matmul_dev(dummy.ptr, dummy.ptr, dc.ptr, m, 0, n, stream=s)
        gr = backend.graph_end(s)
        for _ in range(3):
            dc.upload(np.full(m * n, 7.0, np.float32))
            backend.graph_launch(gr, s)
            backend.synchronize()
            assert np.array_equal(dc.download(np.float32, m * n), np.zeros(m * n, np.float32))
        backend.graph_release(gr)
    finally:
        dc.close()
        dummy.close()

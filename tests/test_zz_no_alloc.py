"""The no-allocation entry point (realm_hip_weights_matmul_noalloc_dev)
through the C ABI against realm_hip_weights_matmul_dev on the same resident
weights and inputs: two calls in a row (the second with a smaller input) on
the integer-dot GEMV, the small-batch MFMA tile and the LDS-tiled kernel with
K splits (bit-identical: same kernels, same splits), one product whose K
splits are reduced to fit the fixed scratch (within 1e-3 relative L2), the
oversize rejection, and that the stream's own scratch never grows meanwhile.
"""
from ctypes import c_void_p

import numpy as np
import pytest

from realm_amd import synth
from realm_amd.formats import GGML_Q4_K, GGML_Q6_K

from conftest import rel_l2

pytestmark = pytest.mark.gpu

INVALID_ARGUMENT = 3


def _noalloc(backend, h, d_x, m, d_y, stream):
    return backend.lib.realm_hip_weights_matmul_noalloc_dev(h, c_void_p(d_x), m, c_void_p(d_y),
                                                            c_void_p(stream))


def _pair(backend, t, n, k, ms, seed):
    """For each m in ms (in order, on one stream): the no-allocation call and
    the regular one on the same input; returns [(noalloc, regular, kernel)]."""
    g = synth.rng(seed)
    blocks = synth.blocks(g, t, n, k)
    h = backend.register_weights(t, blocks, n, k)
    s = backend.stream()
    mmax = max(ms)
    dx = backend.alloc(mmax * k * 4)
    dy0, dy1 = backend.alloc(mmax * n * 4), backend.alloc(mmax * n * 4)
    out = []
    try:
        for m in ms:
            dx.upload(synth.activations(g, m, k))
            dy0.upload(np.full(m * n, np.nan, np.float32))
            before = backend.workspace_info(s)[0]
            assert _noalloc(backend, h, dx.ptr, m, dy0.ptr, s) == 0, backend.last_error()
            kernel = backend.last_kernel()
            backend.synchronize()
            assert backend.workspace_info(s)[0] == before  # nothing allocated
            a = dy0.download(np.float32, m * n)
            backend.matmul_dev(h, dx.ptr, m, dy1.ptr, stream=s)
            backend.synchronize()
            out.append((a, dy1.download(np.float32, m * n), kernel))
    finally:
        backend.release_weights(h)
        for d in (dx, dy0, dy1):
            d.close()
    return out


@pytest.mark.parametrize("t,n,k,ms,prefix", [
    (GGML_Q4_K, 1024, 4096, (200, 37), "realm_gemm_tiled_reduce"),  # tiled, K splits
    (GGML_Q6_K, 600, 2048, (70, 16), "realm_gemm_tiled_reduce"),
    (GGML_Q4_K, 512, 4096, (4, 3), "realm_gemv_q4k"),              # no scratch at all
    (GGML_Q4_K, 700, 1536, (8, 5), "realm_gemm_q4k_s1"),           # small-batch tile
])
def test_noalloc_matches_regular(backend, t, n, k, ms, prefix):
    for m, (a, b, kernel) in zip(ms, _pair(backend, t, n, k, ms, 9000 + n)):
        assert kernel.startswith(prefix), kernel
        assert np.isfinite(a).all()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (m, kernel)


def test_noalloc_reduced_splits(backend):
    """900 tokens x K = 7168: the staging takes 27 MB of the 32 MiB, so the
    tiled launch's two K splits (7.6 MB of parts) drop to one; the result
    matches the regular product to f32 rounding; then a smaller call."""
    res = _pair(backend, GGML_Q4_K, 1024, 7168, (900, 300), 9100)
    assert res[0][2] == "realm_gemm_q4k_t4112p2", res[0][2]  # one split: no reduce launch
    assert res[1][2] == "realm_gemm_tiled_reduce", res[1][2]  # 300 tokens: splits fit
    for a, b, _ in res:
        assert np.isfinite(a).all()
        assert rel_l2(a, b) < 1e-5
    assert np.array_equal(res[1][0].view(np.uint32), res[1][1].view(np.uint32))


def test_noalloc_rejects_oversize(backend):
    n, k, m = 256, 8192, 2000  # staging of 2000 x 8192 f32 tokens: about 70 MB
    g = synth.rng(9200)
    h = backend.register_weights(GGML_Q4_K, synth.blocks(g, GGML_Q4_K, n, k), n, k)
    s = backend.stream()
    dx, dy = backend.alloc(m * k * 4), backend.alloc(m * n * 4)
    try:
        before = backend.workspace_info(s)[0]
        rc = _noalloc(backend, h, dx.ptr, m, dy.ptr, s)
        assert rc == INVALID_ARGUMENT, rc
        assert "no-allocation" in backend.last_error()
        assert backend.workspace_info(s)[0] == before
        assert _noalloc(backend, h, dx.ptr, m, dy.ptr, 0) == INVALID_ARGUMENT  # no stream
    finally:
        backend.release_weights(h)
        dx.close()
        dy.close()

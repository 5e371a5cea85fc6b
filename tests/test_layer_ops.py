"""RMSNorm (with the fused residual add) and SwiGLU: the oracle's numpy
restatement pinned by closed forms and an fp64 brute force (CPU), and the
HIP kernels through the C ABI against it (GPU)."""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import layer_ops as lo


# --------------------------------------------------------------- oracle

def test_oracle_rms_norm_closed_forms():
    w = np.ones(64, np.float32)
    y, _ = lo.rms_norm(np.full((1, 64), -3.0, np.float32), w, 0.0)
    assert np.allclose(y, -1.0, rtol=1e-6)                 # constant row -> sign
    y, _ = lo.rms_norm(np.zeros((2, 64), np.float32), w, 1e-5)
    assert np.array_equal(y, np.zeros((2, 64), np.float32))  # zero row -> 0 (eps > 0)
    g = np.random.default_rng(0)
    x = g.standard_normal((3, 256)).astype(np.float32)
    w256 = np.ones(256, np.float32)
    a, _ = lo.rms_norm(x, w256, 0.0)
    b, _ = lo.rms_norm(x * np.float32(1024.0), w256, 0.0)
    assert np.allclose(a, b, rtol=1e-5)                    # scale invariance (eps = 0)
    wt = g.standard_normal(256).astype(np.float32)
    r = g.standard_normal((3, 256)).astype(np.float32)
    got, h = lo.rms_norm(x, wt, 1e-6, residual=r)
    h64 = x.astype(np.float64) + r
    want = h64 / np.sqrt(np.mean(h64 * h64, axis=1, keepdims=True) + 1e-6) * wt
    assert np.array_equal(h, (x + r).astype(np.float32))
    assert rel_l2(got, want) < 1e-6                         # fp64 brute force


def test_oracle_swiglu_closed_forms():
    u = np.array([2.0, 3.0, -1.0, 5.0], np.float32)
    out = lo.swiglu(np.array([0.0, 50.0, -50.0, 1.0], np.float32), u)
    assert out[0] == 0.0                                   # silu(0) = 0
    assert out[1] == np.float32(150.0)                     # silu(g) -> g for large g
    assert abs(out[2]) < 1e-18                              # silu(g) -> 0 for very negative g
    assert np.isclose(out[3], 5.0 / (1.0 + np.exp(-1.0)), rtol=1e-6)


# ------------------------------------------------------------------ GPU

@pytest.mark.gpu
@pytest.mark.parametrize("rows,hidden", [(1, 4096), (7, 8192), (64, 4096), (3, 100), (2, 28672)])
def test_rms_norm(backend, rows, hidden):
    """RMSNorm alone, fused with the residual (sum written out), and in place."""
    g = np.random.default_rng(rows * 1000 + hidden)
    x = (g.standard_normal((rows, hidden)) * 3).astype(np.float32)
    r = g.standard_normal((rows, hidden)).astype(np.float32)
    w = (1 + 0.1 * g.standard_normal(hidden)).astype(np.float32)
    eps = 1e-5
    dx, dr, dw = (backend.alloc(a.nbytes).upload(a) for a in (x, r, w))
    dy, ds = backend.alloc(x.nbytes), backend.alloc(x.nbytes)
    try:
        backend.rms_norm_dev(dx.ptr, dw.ptr, eps, rows, hidden, dy.ptr)
        backend.synchronize()
        want, _ = lo.rms_norm(x, w, eps)
        assert rel_l2(dy.download(np.float32, x.size).reshape(x.shape), want) < 1e-6
        backend.rms_norm_dev(dx.ptr, dw.ptr, eps, rows, hidden, dy.ptr, d_residual=dr.ptr,
                             d_sum=ds.ptr)
        backend.synchronize()
        want, h = lo.rms_norm(x, w, eps, residual=r)
        assert np.array_equal(ds.download(np.float32, x.size).reshape(x.shape), h)
        assert rel_l2(dy.download(np.float32, x.size).reshape(x.shape), want) < 1e-6
        backend.rms_norm_dev(dx.ptr, dw.ptr, eps, rows, hidden, dx.ptr)  # in place
        backend.synchronize()
        want, _ = lo.rms_norm(x, w, eps)
        assert rel_l2(dx.download(np.float32, x.size).reshape(x.shape), want) < 1e-6
    finally:
        for b in (dx, dr, dw, dy, ds):
            b.close()


@pytest.mark.gpu
@pytest.mark.parametrize("n", [4, 11008, 32 * 28672])
def test_swiglu(backend, n):
    g = np.random.default_rng(n)
    gate = (g.standard_normal(n) * 4).astype(np.float32)
    gate[:4] = [0.0, 60.0, -60.0, 1e-30][: min(4, n)]
    up = g.standard_normal(n).astype(np.float32)
    dg, du = backend.alloc(gate.nbytes).upload(gate), backend.alloc(up.nbytes).upload(up)
    do = backend.alloc(gate.nbytes)
    try:
        backend.swiglu_dev(dg.ptr, du.ptr, n, do.ptr)
        backend.synchronize()
        want = lo.swiglu(gate, up)
        got = do.download(np.float32, n)
        assert np.allclose(got, want, rtol=2e-6, atol=1e-30)
        backend.swiglu_dev(dg.ptr, du.ptr, n, dg.ptr)  # in place over the gate
        backend.synchronize()
        assert np.allclose(dg.download(np.float32, n), want, rtol=2e-6, atol=1e-30)
    finally:
        for b in (dg, du, do):
            b.close()


@pytest.mark.gpu
def test_layer_op_argument_checks(backend):
    from realm_amd.backend import InvalidShape
    d = backend.alloc(4096)
    try:
        with pytest.raises(InvalidShape):
            backend.rms_norm_dev(d.ptr, d.ptr, 1e-5, 1, 6, d.ptr)        # hidden % 4
        with pytest.raises(InvalidShape):
            backend.rms_norm_dev(d.ptr + 4, d.ptr, 1e-5, 1, 8, d.ptr)    # misaligned
        with pytest.raises(InvalidShape):
            backend.rms_norm_dev(d.ptr, d.ptr, 1e-5, 1, 8, d.ptr, d_residual=d.ptr + 64,
                                 d_sum=d.ptr)                            # sum over x
        with pytest.raises(InvalidShape):
            backend.swiglu_dev(d.ptr, d.ptr, 6, d.ptr)
    finally:
        d.close()

"""RoPE, the KV-cache append and causal GQA attention: the oracle's numpy
restatement pinned by closed forms and an fp64 brute force (CPU), the HIP
kernels through the C ABI against it (GPU)."""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import attention as oa


def _fp64_attention(q, k, v, seq_len, kv_len, position, heads, kv_heads, hd):
    q = q.reshape(seq_len, heads, hd).astype(np.float64)
    k = k.reshape(kv_len, kv_heads, hd).astype(np.float64)
    v = v.reshape(kv_len, kv_heads, hd).astype(np.float64)
    out = np.zeros((seq_len, heads, hd))
    for i in range(seq_len):
        for h in range(heads):
            kh = h // (heads // kv_heads)
            vis = min(kv_len, position + i + 1)
            s = k[:vis, kh] @ q[i, h] / np.sqrt(hd)
            p = np.exp(s - s.max())
            out[i, h] = (p / p.sum()) @ v[:vis, kh]
    return out.reshape(-1)


# --------------------------------------------------------------- oracle

def test_oracle_rope_closed_forms():
    g = np.random.default_rng(0)
    x = g.standard_normal(2 * 4 * 64).astype(np.float32)
    assert np.array_equal(oa.rope(x[:256], 0, 1, 4, 64, 10000.0), x[:256])  # position 0
    y = oa.rope(x, 5, 2, 4, 64, 10000.0).reshape(-1, 2)
    assert np.allclose(np.hypot(y[:, 0], y[:, 1]), np.hypot(*x.reshape(-1, 2).T), rtol=1e-5)
    # pair 0 (freq 1) of position p rotates by p radians
    z = oa.rope(np.array([1.0, 0.0] * 32, np.float32), 3, 1, 1, 64, 10000.0)
    assert np.allclose(z[:2], [np.cos(3.0), np.sin(3.0)], atol=1e-6)


def test_oracle_attention_closed_forms_and_fp64():
    g = np.random.default_rng(1)
    hd, heads, kvh = 64, 8, 2
    q = g.standard_normal(heads * hd).astype(np.float32)
    k = g.standard_normal(kvh * hd).astype(np.float32)
    v = g.standard_normal(kvh * hd).astype(np.float32)
    out = oa.attention(q, k, v, 1, 1, 0, heads, kvh, hd).reshape(heads, hd)
    assert np.array_equal(out, np.repeat(v.reshape(kvh, hd), heads // kvh, axis=0))  # one key
    kk = np.tile(k, 5)                      # five equal keys: uniform weights
    vv = g.standard_normal(5 * kvh * hd).astype(np.float32)
    out = oa.attention(q, kk, vv, 1, 5, 4, heads, kvh, hd).reshape(heads, hd)
    want = np.repeat(vv.reshape(5, kvh, hd).mean(0), heads // kvh, axis=0)
    assert np.allclose(out, want, rtol=1e-5, atol=1e-6)
    for seq, kv, pos in ((3, 10, 7), (4, 4, 0), (1, 33, 32)):
        q = g.standard_normal(seq * heads * hd).astype(np.float32)
        k = g.standard_normal(kv * kvh * hd).astype(np.float32)
        v = g.standard_normal(kv * kvh * hd).astype(np.float32)
        got = oa.attention(q, k, v, seq, kv, pos, heads, kvh, hd)
        assert rel_l2(got, _fp64_attention(q, k, v, seq, kv, pos, heads, kvh, hd)) < 1e-5


def test_oracle_kv_append_overflow():
    kc, vc = np.zeros(4 * 8, np.float32), np.zeros(4 * 8, np.float32)
    n = oa.kv_append(kc, vc, 0, 4, np.ones(24, np.float32), np.ones(24, np.float32), 8)
    assert n == 3 and kc[:24].sum() == 24 and kc[24:].sum() == 0
    with pytest.raises(oa.KVCacheError):
        oa.kv_append(kc, vc, 3, 4, np.ones(16, np.float32), np.ones(16, np.float32), 8)


# ------------------------------------------------------------------ GPU

@pytest.mark.gpu
@pytest.mark.parametrize("seq,heads,hd,start", [(1, 32, 128, 0), (1, 32, 128, 4095),
                                                (5, 8, 64, 17), (3, 64, 128, 100)])
def test_rope(backend, seq, heads, hd, start):
    g = np.random.default_rng(seq * 100 + start)
    x = g.standard_normal(seq * heads * hd).astype(np.float32)
    d = backend.alloc(x.nbytes).upload(x)
    try:
        backend.rope_dev(d.ptr, seq, heads, hd, start, 10000.0)
        backend.synchronize()
        got = d.download(np.float32, x.size)
    finally:
        d.close()
    want = oa.rope(x, start, seq, heads, hd, 10000.0)
    # a 1-ulp difference between two libms' powf in freq moves the f32 angle
    # by position x 2^-23 relative: the bound is 2 such ulps at the largest
    # position (the reference's Rust powf has the same freedom)
    tol = 1e-5 + 2.4e-7 * (start + seq)
    assert np.allclose(got, want, rtol=0, atol=tol * np.abs(x).max())
    assert rel_l2(got, want) < tol


@pytest.mark.gpu
@pytest.mark.parametrize("seq,kv,pos,heads,kvh,hd", [
    (1, 1, 0, 32, 32, 128),        # first decode token
    (1, 300, 299, 32, 8, 128),     # decode with GQA (LLaMA-70B head ratio)
    (1, 2048, 2047, 32, 32, 128),  # long context
    (7, 7, 0, 8, 2, 64),           # prefill chunk from empty
    (5, 20, 15, 16, 4, 64),        # prefill chunk after 15 cached tokens
    (3, 40, 10, 4, 4, 256),        # cache longer than the visible keys
])
@pytest.mark.parametrize("splits", ["", "1", "3", "16"])
def test_attention(backend, monkeypatch, seq, kv, pos, heads, kvh, hd, splits):
    """The one-workgroup form and the split-K form (partials, then a
    combine) with its default and forced split counts, including splits
    with no visible keys (3 and 16 splits of short caches)."""
    if splits:
        monkeypatch.setenv("REALM_ATT_SPLITS", splits)
    g = np.random.default_rng(seq * 7 + kv)
    q = g.standard_normal(seq * heads * hd).astype(np.float32)
    k = g.standard_normal(kv * kvh * hd).astype(np.float32)
    v = g.standard_normal(kv * kvh * hd).astype(np.float32)
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
    assert rel_l2(got, want) < 1e-5


TILED_CASES = [  # (seq, kv, pos, heads, kv heads, head_dim, forced tiled, forced splits)
    (511, 511, 0, 32, 32, 128, None, None),   # the bench prefill chunk (16 query tiles)
    (70, 100, 30, 8, 2, 128, None, "1"),      # partial tiles, GQA, cache past the visible keys
    (70, 100, 30, 8, 2, 128, None, "3"),      # the same over 3 key splits
    (33, 33, 0, 4, 4, 32, None, None),        # one query past a tile
    (16, 4000, 3984, 4, 1, 256, None, None),  # long cache: 32 splits of 4 blocks
    (16, 4000, 3984, 4, 1, 256, None, "1"),   # the same walked by one workgroup per head
    (40, 300, 100, 8, 4, 64, None, "7"),      # splits past the visible keys
    (5, 20, 15, 16, 4, 64, "1", None),        # forced below its default threshold
    (1, 40, 39, 2, 2, 64, "1", "1"),          # one token
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", TILED_CASES, ids=[f"s{c[0]}-kv{c[1]}-hd{c[5]}-t{c[6]}-ks{c[7]}" for c in TILED_CASES])
def test_attention_tiled(backend, monkeypatch, case):
    """The tiled prefill form (32 queries x 32 keys per step on f32 MFMA,
    online softmax; keys split over workgroups and combined when the query
    tiles are few) against the oracle, with the one-workgroup-per-token
    form on the same inputs as a second check."""
    seq, kv, pos, heads, kvh, hd, force, ks = case
    if force:
        monkeypatch.setenv("REALM_ATT_TILED", force)
    if ks:
        monkeypatch.setenv("REALM_ATT_TSPLITS", ks)
    g = np.random.default_rng(seq * 11 + kv)
    q = g.standard_normal(seq * heads * hd).astype(np.float32)
    k = g.standard_normal(kv * kvh * hd).astype(np.float32)
    v = g.standard_normal(kv * kvh * hd).astype(np.float32)
    dq, dk, dv = (backend.alloc(a.nbytes).upload(a) for a in (q, k, v))
    do = backend.alloc(q.nbytes)
    try:
        backend.attention_dev(dq.ptr, dk.ptr, dv.ptr, seq, kv, pos, heads, kvh, hd, do.ptr)
        backend.synchronize()
        kernel = backend.last_kernel()
        got = do.download(np.float32, q.size)
        monkeypatch.setenv("REALM_ATT_TILED", "0")
        backend.attention_dev(dq.ptr, dk.ptr, dv.ptr, seq, kv, pos, heads, kvh, hd, do.ptr)
        backend.synchronize()
        other = do.download(np.float32, q.size)
    finally:
        for b in (dq, dk, dv, do):
            b.close()
    if ks == "1":
        assert kernel == f"realm_attention_tiled_h{hd}"
    else:
        assert kernel in (f"realm_attention_tiled_h{hd}", "realm_attention_combine")
    want = oa.attention(q, k, v, seq, kv, pos, heads, kvh, hd)
    assert rel_l2(got, want) < 1e-5
    assert rel_l2(got, other) < 1e-5


@pytest.mark.gpu
def test_attention_split_graph_replays(backend):
    """The split form (8 splits at this decode shape, then the combine)
    captured once and replayed three times, with eager launches on the same
    stream in between, every replay against the oracle."""
    seq, kv, pos, heads, kvh, hd = 1, 512, 511, 32, 32, 128
    g = np.random.default_rng(5)
    q = g.standard_normal(seq * heads * hd).astype(np.float32)
    k = g.standard_normal(kv * kvh * hd).astype(np.float32)
    v = g.standard_normal(kv * kvh * hd).astype(np.float32)
    want = oa.attention(q, k, v, seq, kv, pos, heads, kvh, hd)
    dq, dk, dv = (backend.alloc(a.nbytes).upload(a) for a in (q, k, v))
    do, de = backend.alloc(q.nbytes), backend.alloc(q.nbytes)
    s = backend.stream()
    run = lambda out: backend.attention_dev(dq.ptr, dk.ptr, dv.ptr, seq, kv, pos, heads, kvh, hd,
                                            out.ptr, stream=s)
    try:
        run(do)
        backend.synchronize()
        assert backend.last_kernel() == "realm_attention_combine"
        backend.graph_begin(s)
        run(do)
        gr = backend.graph_end(s)
        try:
            for _ in range(3):
                do.upload(np.zeros(q.size, np.float32))
                backend.graph_launch(gr, s)
                backend.synchronize()
                assert rel_l2(do.download(np.float32, q.size), want) < 1e-5
                run(de)  # eager launch between replays, same scratch
                backend.synchronize()
                assert rel_l2(de.download(np.float32, q.size), want) < 1e-5
        finally:
            backend.graph_release(gr)
    finally:
        for b in (dq, dk, dv, do, de):
            b.close()


@pytest.mark.gpu
def test_kv_append_then_attention(backend):
    """Decode three steps into a device cache (append, then attend) against
    the oracle's cache; the overflowing append fails with ParseError (4)."""
    from realm_amd.backend import RealmError
    heads, kvh, hd, max_len = 8, 2, 64, 6
    kv_dim = kvh * hd
    g = np.random.default_rng(3)
    kc_ref, vc_ref = np.zeros(max_len * kv_dim, np.float32), np.zeros(max_len * kv_dim, np.float32)
    dkc, dvc = backend.alloc(kc_ref.nbytes), backend.alloc(vc_ref.nbytes)
    cur = 0
    try:
        for step, n in enumerate((3, 1, 2)):
            k = g.standard_normal(n * kv_dim).astype(np.float32)
            v = g.standard_normal(n * kv_dim).astype(np.float32)
            q = g.standard_normal(n * heads * hd).astype(np.float32)
            dk, dv, dq = (backend.alloc(a.nbytes).upload(a) for a in (k, v, q))
            do = backend.alloc(q.nbytes)
            backend.kv_append_dev(dk.ptr, dv.ptr, n, kv_dim, cur, max_len, dkc.ptr, dvc.ptr)
            new = oa.kv_append(kc_ref, vc_ref, cur, max_len, k, v, kv_dim)
            backend.attention_dev(dq.ptr, dkc.ptr, dvc.ptr, n, new, cur, heads, kvh, hd, do.ptr)
            backend.synchronize()
            want = oa.attention(q, kc_ref[:new * kv_dim], vc_ref[:new * kv_dim], n, new, cur,
                                heads, kvh, hd)
            assert rel_l2(do.download(np.float32, q.size), want) < 1e-5, step
            cur = new
            for b in (dk, dv, dq, do):
                b.close()
        with pytest.raises(RealmError) as e:
            backend.kv_append_dev(dkc.ptr, dvc.ptr, 1, kv_dim, cur, max_len, dkc.ptr, dvc.ptr)
        assert e.value.code == 4
    finally:
        dkc.close()
        dvc.close()


@pytest.mark.gpu
@pytest.mark.parametrize("fuse", ["1", "0", "rope"])
@pytest.mark.parametrize("mixed", [False, True])
def test_forward_layer(backend, oracle, monkeypatch, mixed, fuse):
    """realm_hip_forward_layer_dev against the oracle's composition of the
    reference's steps: a 5-token prefill from an empty cache, a 1-token and
    a 3-token decode after it (the GEMV and MFMA product paths), and a call
    that would overflow the cache.  mixed: V and up in Q6_K (separate
    products), otherwise every projection in Q4_K (grouped products).  The
    1-token call runs with the norms and SwiGLU fused into the GEMVs
    (fuse "1", where the formats allow), as separate launches ("0"), and
    fused with the split attention forced ("rope": RoPE of q and of the new
    key row inside the attention kernel, which writes the rotated row into
    the cache)."""
    monkeypatch.setenv("REALM_LAYER_FUSE", "0" if fuse == "0" else "1")
    if fuse == "rope":
        monkeypatch.setenv("REALM_ATT_SPLITS", "2")
    from realm_amd import synth
    from realm_amd.backend import RealmError, RealmLayer
    from realm_amd.formats import GGML_Q4_K, GGML_Q6_K
    H, heads, kvh, hd, inter, max_len = 256, 4, 2, 64, 512, 12
    kv_dim = kvh * hd
    cfg = {"hidden": H, "heads": heads, "kv_heads": kvh, "head_dim": hd, "eps": 1e-5,
           "theta": 10000.0}
    g = synth.rng(40 + mixed)
    shapes = {"wq": (H, H), "wk": (kv_dim, H), "wv": (kv_dim, H), "wo": (H, H),
              "w_gate": (inter, H), "w_up": (inter, H), "w_down": (H, inter)}
    types = {name: GGML_Q4_K for name in shapes}
    if mixed:
        types["wv"] = types["w_up"] = GGML_Q6_K
    blocks = {name: synth.blocks(g, types[name], n, k) for name, (n, k) in shapes.items()}
    # larger scales than the synthetic 1e-3 so that every step matters
    for b in blocks.values():
        b["d"] = (b["d"].view(np.float16) * np.float16(40)).view(np.uint16)
    handles = {name: backend.register_weights(types[name], blocks[name], *shapes[name])
               for name in shapes}
    norms = {"attn": (1 + 0.1 * g.standard_normal(H)).astype(np.float32),
             "ffn": (1 + 0.1 * g.standard_normal(H)).astype(np.float32)}
    dn = {key: backend.alloc(v.nbytes).upload(v) for key, v in norms.items()}
    layer = RealmLayer(wq=handles["wq"], wk=handles["wk"], wv=handles["wv"], wo=handles["wo"],
                       w_gate=handles["w_gate"], w_up=handles["w_up"], w_down=handles["w_down"],
                       attn_norm=dn["attn"].ptr, ffn_norm=dn["ffn"].ptr, hidden=H,
                       num_heads=heads, num_kv_heads=kvh, head_dim=hd, intermediate=inter,
                       rms_norm_eps=1e-5, rope_theta=10000.0)

    def matmul(name, x, m):
        n, k = shapes[name]
        rc, y = oracle.candle_fused(types[name], blocks[name], np.ascontiguousarray(x), m, n, k)
        assert rc == 0
        return y.reshape(m, n)

    kc_ref = np.zeros(max_len * kv_dim, np.float32)
    vc_ref = np.zeros(max_len * kv_dim, np.float32)
    dkc, dvc = backend.alloc(kc_ref.nbytes), backend.alloc(vc_ref.nbytes)
    pos = 0
    try:
        for seq in (5, 1, 3):
            x = g.standard_normal((seq, H)).astype(np.float32)
            dx, dy = backend.alloc(x.nbytes).upload(x), backend.alloc(x.nbytes)
            backend.forward_layer_dev(layer, dx.ptr, seq, pos, dkc.ptr, dvc.ptr, max_len, dy.ptr)
            backend.synchronize()
            got = dy.download(np.float32, x.size).reshape(seq, H)
            want = forward = oa.forward_layer(matmul, x, blocks, norms, cfg, kc_ref, vc_ref, pos,
                                              seq)
            err = rel_l2(got, want)
            delta = rel_l2(got - x, forward - x)  # the layer's own contribution
            print(f"forward_layer mixed={mixed} seq={seq} pos={pos} rel_l2={err:.3e} "
                  f"delta={delta:.3e}")
            assert err < 1e-3 and delta < 1e-3, (seq, pos)
            kc = dkc.download(np.float32, kc_ref.size)
            assert rel_l2(kc[:(pos + seq) * kv_dim], kc_ref[:(pos + seq) * kv_dim]) < 1e-3
            pos += seq
            dx.close()
            dy.close()
        x = np.zeros((4, H), np.float32)
        dx, dy = backend.alloc(x.nbytes).upload(x), backend.alloc(x.nbytes)
        with pytest.raises(RealmError) as e:
            backend.forward_layer_dev(layer, dx.ptr, 4, pos, dkc.ptr, dvc.ptr, max_len, dy.ptr)
        assert e.value.code == 4
        dx.close()
        dy.close()
    finally:
        for h in handles.values():
            backend.release_weights(h)
        for b in list(dn.values()) + [dkc, dvc]:
            b.close()


@pytest.mark.gpu
@pytest.mark.parametrize("fuse", ["1", "0", "rope"])
def test_forward_layers_chain(backend, oracle, monkeypatch, fuse):
    """Three layers in one realm_hip_forward_layers_dev call (the residual add
    fused into the next layer's first norm) against three oracle layers
    applied in turn, for a 4-token prefill and a 1-token decode after it
    (fuse "1": the decode's norms, residual adds and SwiGLU inside the
    GEMVs; "0": separate launches; "rope": fused, with the split attention
    forced, RoPE inside it)."""
    monkeypatch.setenv("REALM_LAYER_FUSE", "0" if fuse == "0" else "1")
    if fuse == "rope":
        monkeypatch.setenv("REALM_ATT_SPLITS", "2")
    from realm_amd import synth
    from realm_amd.backend import RealmLayer
    from realm_amd.formats import GGML_Q4_K, GGML_Q6_K
    H, heads, kvh, hd, inter, max_len, nl = 256, 4, 2, 64, 512, 8, 3
    kv_dim = kvh * hd
    cfg = {"hidden": H, "heads": heads, "kv_heads": kvh, "head_dim": hd, "eps": 1e-5,
           "theta": 10000.0}
    shapes = {"wq": (H, H), "wk": (kv_dim, H), "wv": (kv_dim, H), "wo": (H, H),
              "w_gate": (inter, H), "w_up": (inter, H), "w_down": (H, inter)}
    g = synth.rng(77)
    per, layers, bufs, handles = [], [], [], []
    for li in range(nl):
        types = {n: (GGML_Q6_K if n == "w_down" else GGML_Q4_K) for n in shapes}
        blocks = {n: synth.blocks(g, types[n], *shapes[n]) for n in shapes}
        for b in blocks.values():
            b["d"] = (b["d"].view(np.float16) * np.float16(40)).view(np.uint16)
        hs = {n: backend.register_weights(types[n], blocks[n], *shapes[n]) for n in shapes}
        handles += hs.values()
        norms = {"attn": (1 + 0.1 * g.standard_normal(H)).astype(np.float32),
                 "ffn": (1 + 0.1 * g.standard_normal(H)).astype(np.float32)}
        dn = {k: backend.alloc(v.nbytes).upload(v) for k, v in norms.items()}
        kc, vc = backend.alloc(max_len * kv_dim * 4), backend.alloc(max_len * kv_dim * 4)
        bufs += list(dn.values()) + [kc, vc]
        layers.append(RealmLayer(wq=hs["wq"], wk=hs["wk"], wv=hs["wv"], wo=hs["wo"],
                                 w_gate=hs["w_gate"], w_up=hs["w_up"], w_down=hs["w_down"],
                                 attn_norm=dn["attn"].ptr, ffn_norm=dn["ffn"].ptr, hidden=H,
                                 num_heads=heads, num_kv_heads=kvh, head_dim=hd,
                                 intermediate=inter, rms_norm_eps=1e-5, rope_theta=10000.0))
        per.append((types, blocks, norms, np.zeros(max_len * kv_dim, np.float32),
                    np.zeros(max_len * kv_dim, np.float32), kc, vc))
    try:
        pos = 0
        for seq in (4, 1):
            x = g.standard_normal((seq, H)).astype(np.float32)
            dx, dy = backend.alloc(x.nbytes).upload(x), backend.alloc(x.nbytes)
            backend.forward_layers_dev(layers, dx.ptr, seq, pos, [p[5].ptr for p in per],
                                       [p[6].ptr for p in per], max_len, dy.ptr)
            backend.synchronize()
            got = dy.download(np.float32, x.size).reshape(seq, H)
            want = x
            for types, blocks, norms, kr, vr, _, _ in per:
                def matmul(name, a, m, types=types, blocks=blocks):
                    n, k = shapes[name]
                    rc, y = oracle.candle_fused(types[name], blocks[name],
                                                np.ascontiguousarray(a), m, n, k)
                    assert rc == 0
                    return y.reshape(m, n)
                want = oa.forward_layer(matmul, want, blocks, norms, cfg, kr, vr, pos, seq)
            err = rel_l2(got, want)
            print(f"forward_layers seq={seq} pos={pos} rel_l2={err:.3e}")
            assert err < 1e-3, (seq, pos)
            pos += seq
            dx.close()
            dy.close()
    finally:
        for h in handles:
            backend.release_weights(h)
        for b in bufs:
            b.close()


@pytest.mark.gpu
@pytest.mark.parametrize("which", ["all", "some"])
def test_forward_layer_lora(backend, oracle, which):
    """Per-tenant LoRA inside realm_hip_forward_layer_dev: adapter sets on all
    seven projections (grouped multi-LoRA products for q/k/v and gate/up), or
    on q, v, o and down only (per-projection products where a group is
    mixed); tokens of three tenants, one without adapter (-1) and one past
    the sets' size (base only); a 6-token prefill, then a 1- and a 2-token
    decode.  Against the oracle's composition of the reference's steps with
    each projection's product y = W x + s B (A x) (lora.rs:91-144 unmerged),
    on every token."""
    from realm_amd import synth
    from realm_amd.backend import RealmLayer
    from realm_amd.formats import GGML_Q4_K, GGML_Q6_K
    H, heads, kvh, hd, inter, max_len = 256, 4, 2, 64, 512, 12
    kv_dim = kvh * hd
    cfg = {"hidden": H, "heads": heads, "kv_heads": kvh, "head_dim": hd, "eps": 1e-5,
           "theta": 10000.0}
    g = synth.rng(90 + (which == "some"))
    shapes = {"wq": (H, H), "wk": (kv_dim, H), "wv": (kv_dim, H), "wo": (H, H),
              "w_gate": (inter, H), "w_up": (inter, H), "w_down": (H, inter)}
    types = {name: (GGML_Q6_K if name == "w_down" else GGML_Q4_K) for name in shapes}
    blocks = {name: synth.blocks(g, types[name], n, k) for name, (n, k) in shapes.items()}
    for b in blocks.values():
        b["d"] = (b["d"].view(np.float16) * np.float16(40)).view(np.uint16)
    handles = {name: backend.register_weights(types[name], blocks[name], *shapes[name])
               for name in shapes}
    with_lora = list(shapes) if which == "all" else ["wq", "wv", "wo", "w_down"]
    adapters, sets, lhs = {}, {}, []
    for name in with_lora:
        n, k = shapes[name]
        ads = []
        for r in (4, 16):  # two tenants with adapters on this projection
            a, b = synth.lora_adapter(g, r, k, n)
            b = (b.astype(np.float32) * 20).astype(np.float16)  # deltas that matter
            ads.append((a, b, r, 16.0))
        hs = [backend.lora_register(a, b, r, al, k, n) for a, b, r, al in ads]
        lhs += hs
        adapters[name] = ads
        sets[name] = backend.lora_set_create(hs)
    norms = {"attn": (1 + 0.1 * g.standard_normal(H)).astype(np.float32),
             "ffn": (1 + 0.1 * g.standard_normal(H)).astype(np.float32)}
    dn = {key: backend.alloc(v.nbytes).upload(v) for key, v in norms.items()}
    kc_ref = np.zeros(max_len * kv_dim, np.float32)
    vc_ref = np.zeros(max_len * kv_dim, np.float32)
    dkc, dvc = backend.alloc(kc_ref.nbytes), backend.alloc(vc_ref.nbytes)
    pos = 0
    try:
        for seq, ids in ((6, [0, 1, -1, 1, 5, 0]), (1, [1]), (2, [0, -1])):
            ids = np.array(ids, np.int32)
            d_ids = backend.alloc(ids.nbytes).upload(ids)
            layer = RealmLayer(wq=handles["wq"], wk=handles["wk"], wv=handles["wv"],
                               wo=handles["wo"], w_gate=handles["w_gate"], w_up=handles["w_up"],
                               w_down=handles["w_down"], attn_norm=dn["attn"].ptr,
                               ffn_norm=dn["ffn"].ptr, hidden=H, num_heads=heads,
                               num_kv_heads=kvh, head_dim=hd, intermediate=inter,
                               rms_norm_eps=1e-5, rope_theta=10000.0,
                               lora_q=sets.get("wq", 0), lora_k=sets.get("wk", 0),
                               lora_v=sets.get("wv", 0), lora_o=sets.get("wo", 0),
                               lora_gate=sets.get("w_gate", 0), lora_up=sets.get("w_up", 0),
                               lora_down=sets.get("w_down", 0), d_adapter_ids=d_ids.ptr)

            def matmul(name, x, m, ids=ids):
                n, k = shapes[name]
                x = np.ascontiguousarray(x, np.float32)
                rc, y = oracle.candle_fused(types[name], blocks[name], x, m, n, k)
                assert rc == 0
                y = y.reshape(m, n)
                if name in adapters:
                    ad = [(a.astype(np.float32), b.astype(np.float32), r, al)
                          for a, b, r, al in adapters[name]]
                    y = oracle.multi_lora_delta(x, ids, ad, y.copy())
                return y

            x = g.standard_normal((seq, H)).astype(np.float32)
            dx, dy = backend.alloc(x.nbytes).upload(x), backend.alloc(x.nbytes)
            backend.forward_layer_dev(layer, dx.ptr, seq, pos, dkc.ptr, dvc.ptr, max_len, dy.ptr)
            backend.synchronize()
            got = dy.download(np.float32, x.size).reshape(seq, H)
            want = oa.forward_layer(matmul, x, blocks, norms, cfg, kc_ref, vc_ref, pos, seq)
            # the adapters change the output (the check has teeth)
            base = oa.forward_layer(lambda nm, a, m: matmul(nm, a, m, ids=np.full(m, -1, np.int32)),
                                    x, blocks, norms, cfg, kc_ref.copy(), vc_ref.copy(), pos, seq)
            err, change = rel_l2(got, want), rel_l2(want, base)
            print(f"forward_layer lora={which} seq={seq} rel_l2={err:.3e} lora effect={change:.3e}")
            assert err < 1e-3, (seq, pos)
            # the residual dilutes one token's delta at the layer output: the
            # deltas still stand two orders of magnitude above the error
            assert change > 1e-3 and err < change / 100, (seq, change, err)
            pos += seq
            for b in (dx, dy, d_ids):
                b.close()
    finally:
        for s in sets.values():
            backend.lora_set_release(s)
        for h in lhs:
            backend.lora_release(h)
        for h in handles.values():
            backend.release_weights(h)
        for b in list(dn.values()) + [dkc, dvc]:
            b.close()


@pytest.mark.gpu
@pytest.mark.parametrize("seq,kv", [(1, 100_000), (2, 60_001)])
def test_attention_long_cache(backend, seq, kv):
    """Caches longer than one workgroup's LDS holds scores for (about 39 K
    keys): the split form with enough splits that every chunk fits, against
    the oracle (StandardAttention takes any kv_len, standard.rs:36-210)."""
    heads, kvh, hd = 4, 2, 64
    pos = kv - seq
    g = np.random.default_rng(kv)
    q = g.standard_normal(seq * heads * hd).astype(np.float32)
    k = (0.3 * g.standard_normal(kv * kvh * hd)).astype(np.float32)
    v = g.standard_normal(kv * kvh * hd).astype(np.float32)
    dq, dk, dv = (backend.alloc(a.nbytes).upload(a) for a in (q, k, v))
    do = backend.alloc(q.nbytes)
    try:
        backend.attention_dev(dq.ptr, dk.ptr, dv.ptr, seq, kv, pos, heads, kvh, hd, do.ptr)
        backend.synchronize()
        got = do.download(np.float32, q.size)
        assert backend.last_kernel() == "realm_attention_combine"
    finally:
        for b in (dq, dk, dv, do):
            b.close()
    want = oa.attention(q, k, v, seq, kv, pos, heads, kvh, hd)
    assert rel_l2(got, want) < 1e-5


@pytest.mark.gpu
def test_forward_layer_7b_decode_fused(backend, oracle, monkeypatch):
    """One LLaMA-7B-shape layer (hidden 4096, 32 heads of 128, intermediate
    11008; Q4_K projections, Q6_K W_down), the decode step bench.py times:
    a 2-token prefill, then one token with the norms and SwiGLU fused into
    the GEMVs' x staging (the l64 u1 "_n" kernels for Q/K/V and gate/up, the
    u3 "_s" kernel for W_down), the same with the split attention forced
    (RoPE fused into it), and the same token through the separate launches,
    all against the oracle's composition; the K cache row each run writes
    against the oracle's."""
    from realm_amd import synth
    from realm_amd.backend import RealmLayer
    from realm_amd.formats import GGML_Q4_K, GGML_Q6_K
    H, heads, kvh, hd, inter, max_len = 4096, 32, 32, 128, 11008, 4
    kv_dim = kvh * hd
    cfg = {"hidden": H, "heads": heads, "kv_heads": kvh, "head_dim": hd, "eps": 1e-5,
           "theta": 10000.0}
    shapes = {"wq": (H, H), "wk": (kv_dim, H), "wv": (kv_dim, H), "wo": (H, H),
              "w_gate": (inter, H), "w_up": (inter, H), "w_down": (H, inter)}
    types = {n: (GGML_Q6_K if n == "w_down" else GGML_Q4_K) for n in shapes}
    g = synth.rng(4096)
    blocks = {n: synth.blocks(g, types[n], *shapes[n]) for n in shapes}
    for b in blocks.values():
        b["d"] = (b["d"].view(np.float16) * np.float16(8)).view(np.uint16)
    hs = {n: backend.register_weights(types[n], blocks[n], *shapes[n]) for n in shapes}
    norms = {"attn": (1 + 0.1 * g.standard_normal(H)).astype(np.float32),
             "ffn": (1 + 0.1 * g.standard_normal(H)).astype(np.float32)}
    dn = {k: backend.alloc(v.nbytes).upload(v) for k, v in norms.items()}
    layer = RealmLayer(wq=hs["wq"], wk=hs["wk"], wv=hs["wv"], wo=hs["wo"], w_gate=hs["w_gate"],
                       w_up=hs["w_up"], w_down=hs["w_down"], attn_norm=dn["attn"].ptr,
                       ffn_norm=dn["ffn"].ptr, hidden=H, num_heads=heads, num_kv_heads=kvh,
                       head_dim=hd, intermediate=inter, rms_norm_eps=1e-5, rope_theta=10000.0)

    def matmul(name, x, m):
        n, k = shapes[name]
        rc, y = oracle.candle_fused(types[name], blocks[name], np.ascontiguousarray(x), m, n, k)
        assert rc == 0
        return y.reshape(m, n)

    kc_ref = np.zeros(max_len * kv_dim, np.float32)
    vc_ref = np.zeros(max_len * kv_dim, np.float32)
    dkc, dvc = backend.alloc(kc_ref.nbytes), backend.alloc(vc_ref.nbytes)
    bufs = []
    try:
        x0 = g.standard_normal((2, H)).astype(np.float32)
        dx = backend.alloc(x0.nbytes).upload(x0)
        dy = backend.alloc(x0.nbytes)
        bufs += [dx, dy]
        backend.forward_layer_dev(layer, dx.ptr, 2, 0, dkc.ptr, dvc.ptr, max_len, dy.ptr)
        oa.forward_layer(matmul, x0, blocks, norms, cfg, kc_ref, vc_ref, 0, 2)
        x1 = g.standard_normal((1, H)).astype(np.float32)
        want = oa.forward_layer(matmul, x1, blocks, norms, cfg, kc_ref.copy(), vc_ref.copy(), 2, 1)
        d1 = backend.alloc(x1.nbytes).upload(x1)
        bufs.append(d1)
        outs = {}
        kc_want = kc_ref.copy()
        oa.forward_layer(matmul, x1, blocks, norms, cfg, kc_want, vc_ref.copy(), 2, 1)
        for fuse in ("1", "rope", "0"):
            monkeypatch.setenv("REALM_LAYER_FUSE", "0" if fuse == "0" else "1")
            if fuse == "rope":
                monkeypatch.setenv("REALM_ATT_SPLITS", "2")
            else:
                monkeypatch.delenv("REALM_ATT_SPLITS", raising=False)
            do = backend.alloc(x1.nbytes)
            bufs.append(do)
            # the same cache position every time: the step rewrites its K/V row
            backend.forward_layer_dev(layer, d1.ptr, 1, 2, dkc.ptr, dvc.ptr, max_len, do.ptr)
            backend.synchronize()
            outs[fuse] = do.download(np.float32, H).reshape(1, H)
            krow = dkc.download(np.float32, 3 * kv_dim)[2 * kv_dim:]
            assert rel_l2(krow, kc_want[2 * kv_dim:3 * kv_dim]) < 1e-3, fuse
            err = rel_l2(outs[fuse], want)
            delta = rel_l2(outs[fuse] - x1, want - x1)
            print(f"7b decode fuse={fuse} rel_l2={err:.3e} delta={delta:.3e}")
            assert err < 1e-3 and delta < 1e-3, fuse
        assert rel_l2(outs["1"], outs["0"]) < 1e-5
        assert rel_l2(outs["rope"], outs["0"]) < 1e-5
    finally:
        for h in hs.values():
            backend.release_weights(h)
        for b in list(dn.values()) + [dkc, dvc] + bufs:
            b.close()

#!/usr/bin/env python3
"""Benchmark of the MI355X quantized compute path (one GPU).

Headline (the timed region): LLaMA-7B decode, batch 1 -- one step is the
decoder-layer matvec set (Wq, Wk, Wv, Wo, W_gate, W_up in Q4_K, W_down in
Q6_K) of all 32 layers, captured in one HIP graph.  Launches follow the
layer's data dependencies: Q/K/V share their input and go in one grouped
launch, so do gate/up; Wo and W_down each wait for the work before them
(attention and SwiGLU in a full model), so each is a launch of its own: four
launches per layer, 128 per step.  Every layer has its own copy of the
weights in HBM (4.0 GB per step, far beyond the 256 MB Infinity Cache);
activations are resident before timing starts.  ``value`` is algorithmic
GB/s = (packed weight bytes + activations read + outputs written) / step
time; tok/s = batch / step time.

After the timed region, bench.py reports the roofline of the dominant Q4_K
kernel (the grouped gate/up GEMV: its launches replayed from a graph of their
own, HIP events on its stream) and, in "extra": the same step at batch 4 and
16, 16-tenant multi-LoRA overhead (config 3), prefill TFLOP/s (config 2,
Q4_K and Q8_0 with bf16 activations), the config-4 70B-shape layer, the dense
f32 product, the reference's own criterion workloads for the Q4_K fused
kernel (fused_kernels.rs:96-211, with the same shapes timed on the CPU
restatement) and the CPU baseline (the oracle's restatement of
realm-compute-cpu, timed on this host).  All inputs are synthetic and seeded
(realm_amd/synth.py).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

from realm_amd import synth  # noqa: E402
from realm_amd.formats import GGML_Q4_K, GGML_Q6_K, GGML_Q8_0, weight_bytes  # noqa: E402

METRIC = "Q4_K dequant-GEMV HBM GB/s (% peak) + tok/s at 7B; multi-LoRA overhead %"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
LAYERS = 32
LAYER = [("wq", GGML_Q4_K, 4096, 4096), ("wk", GGML_Q4_K, 4096, 4096),
         ("wv", GGML_Q4_K, 4096, 4096), ("wo", GGML_Q4_K, 4096, 4096),
         ("w_gate", GGML_Q4_K, 11008, 4096), ("w_up", GGML_Q4_K, 11008, 4096),
         ("w_down", GGML_Q6_K, 4096, 11008)]


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def alg_bytes(t: int, n: int, k: int, m: int, act_bytes: int = 4) -> int:
    return weight_bytes(t, n, k) + act_bytes * m * k + 4 * m * n


class Model7B:
    """32 layers of distinct device copies of one seeded LLaMA-7B layer."""

    def __init__(self, be, layers: int, max_m: int):
        self.be = be
        g = synth.rng(1)
        host = [(name, t, n, k, synth.blocks(g, t, n, k)) for name, t, n, k in LAYER]
        self.host = {name: b for name, _t, _n, _k, b in host}
        self.layers = []
        for _ in range(layers):
            self.layers.append([(name, t, n, k, be.register_weights(t, b, n, k))
                                for name, t, n, k, b in host])
        self.x_host = {k: synth.activations(g, max_m, k) for k in (4096, 11008)}
        self.x = {k: be.alloc(max_m * k * 4).upload(self.x_host[k]) for k in (4096, 11008)}
        self.y = {name: be.alloc(max_m * n * 4) for name, _, n, _ in LAYER}

    # launch groups of a layer (indices into LAYER): matrices in one group
    # share their input
    GROUPS = ((0, 1, 2), (3,), (4, 5), (6,))

    def launch_group(self, layer, gi: int, m: int, stream: int) -> None:
        idx = self.GROUPS[gi]
        k = LAYER[idx[0]][3]
        hs = [layer[i][4] for i in idx]
        ys = [self.y[LAYER[i][0]].ptr for i in idx]
        if len(hs) == 1:
            self.be.matmul_dev(hs[0], self.x[k].ptr, m, ys[0], stream=stream)
        else:
            self.be.matmul_group_dev(hs, self.x[k].ptr, m, ys, stream=stream)

    def step(self, m: int, stream: int) -> None:
        for layer in self.layers:
            for gi in range(len(self.GROUPS)):
                self.launch_group(layer, gi, m, stream)

    @classmethod
    def group_bytes(cls, gi: int, m: int) -> int:
        """Algorithmic bytes of one launch group: its packed weights, its
        shared input read once, its outputs."""
        idx = cls.GROUPS[gi]
        k = LAYER[idx[0]][3]
        return sum(weight_bytes(LAYER[i][1], LAYER[i][2], k) + 4 * m * LAYER[i][2]
                   for i in idx) + 4 * m * k

    def bytes_per_step(self, m: int) -> int:
        return len(self.layers) * sum(self.group_bytes(gi, m) for gi in range(len(self.GROUPS)))

    def close(self):
        for layer in self.layers:
            for *_, h in layer:
                self.be.release_weights(h)
        for b in list(self.x.values()) + list(self.y.values()):
            b.close()


def capture(be, stream: int, fn) -> int:
    fn()  # eager run sizes the library's scratch buffers
    be.synchronize()
    be.graph_begin(stream)
    fn()
    return be.graph_end(stream)


def time_graph(be, graph: int, stream: int, reps: int) -> float:
    """Mean ms per replay, HIP events on `stream`."""
    e0, e1 = be.event(), be.event()
    be.record(e0, stream)
    for _ in range(reps):
        be.graph_launch(graph, stream)
    be.record(e1, stream)
    return be.elapsed_ms(e0, e1) / reps


ROOF_GROUP = 2  # the grouped gate/up launch: the largest Q4_K kernel of the step
TRAFFIC_FILE = os.path.join(REPO, "profiles", "gemv_q4k_gateup_7b_traffic.json")


def decode_roofline(be, model: Model7B, stream: int, reps: int) -> dict:
    """The dominant Q4_K kernel of the decode step: the grouped gate/up GEMV
    (2 x 11008x4096, batch 1).  Its 32 per-layer launches (distinct weights)
    are replayed from a graph of their own; HIP events on the launch stream
    bracket `reps` replays, so the average includes nothing but those
    kernels back to back.  Algorithmic bytes per launch: both packed
    matrices, x once, both outputs."""
    def launches():
        for layer in model.layers:
            model.launch_group(layer, ROOF_GROUP, 1, stream)
    gr = capture(be, stream, launches)
    kernel = be.last_kernel()
    time_graph(be, gr, stream, 3)
    ms = time_graph(be, gr, stream, reps) / len(model.layers)
    be.graph_release(gr)
    nbytes = Model7B.group_bytes(ROOF_GROUP, 1)
    achieved = nbytes / (ms * 1e-3) / 1e9
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            rec = json.load(f)
        if rec.get("kernel") == kernel:
            traffic = rec.get("hbm_bytes_per_launch")
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": kernel, "launches": len(model.layers) * reps,
            "avg_launch_us": round(ms * 1e3, 3), "alg_bytes_per_launch": nbytes,
            "shape": "grouped W_gate + W_up, 2 x (11008 x 4096) Q4_K, batch 1"}


def stream_ceiling(be, stream: int, reps: int) -> dict:
    """The practical HBM read ceiling, from the library's plain streaming
    kernel (realm_hip_checksum_dev: 16-byte loads, four per lane in flight,
    nothing else) over a separate 4 GB region:
      chain_128: the decode step's launch structure -- 32 layers x the four
        launch groups' byte counts, each launch a checksum of its own slice,
        replayed from one graph (the ceiling for a stream-ordered step);
      gate_up_size: one launch of the roofline kernel's size (the grouped
        gate/up bytes), 32 distinct slices per graph;
      single_4gb: one launch over the whole region."""
    sizes = [Model7B.group_bytes(gi, 1) for gi in range(len(Model7B.GROUPS))]
    sizes = [(s + 255) // 256 * 256 for s in sizes]
    total = LAYERS * sum(sizes)
    buf = be.alloc(total)
    parts = be.alloc(4096 * 4)
    cu = 256
    out = {}

    def run(name, fn, nbytes):
        gr = capture(be, stream, fn)
        time_graph(be, gr, stream, 2)
        ms = time_graph(be, gr, stream, reps)
        be.graph_release(gr)
        out[name] = {"us": round(ms * 1e3, 2), "gb_per_s": round(nbytes / (ms * 1e-3) / 1e9, 1)}

    def chain():
        off = 0
        for _ in range(LAYERS):
            for s in sizes:
                be.checksum_dev(buf.ptr + off, s, parts.ptr, cu, stream=stream)
                off += s
    run("chain_128", chain, total)

    def gate_up():
        for l in range(LAYERS):
            be.checksum_dev(buf.ptr + l * sizes[2], sizes[2], parts.ptr, cu, stream=stream)
    run("gate_up_size", gate_up, LAYERS * sizes[2])
    out["gate_up_size"]["us"] = round(out["gate_up_size"]["us"] / LAYERS, 3)
    run("single_4gb", lambda: be.checksum_dev(buf.ptr, total, parts.ptr, cu, stream=stream), total)
    out["kernel"] = "realm_checksum (1024 threads x 4 x 16 B in flight, one workgroup per CU)"
    buf.close()
    parts.close()
    return out


def full_layers(be, model: Model7B, stream: int, reps: int, context: int = 512) -> dict:
    """The whole decoder layer on the device (realm_hip_forward_layers_dev:
    norm, Q/K/V, RoPE, KV append, attention, Wo, residual + norm, gate/up,
    SwiGLU, W_down, residual; the residual add fused into the next layer's
    first norm) for all of the model's layers in one call, each with its own
    weights and KV cache (LLaMA-7B has 32 KV heads of 128, no GQA): a
    prefill of `context - 1` tokens, then the decode step of the
    next token, each captured in one HIP graph and replayed (every replay
    writes the same cache rows; the decode step attends over `context`
    keys)."""
    from realm_amd.backend import RealmLayer
    H, heads, kvh, hd, inter = 4096, 32, 32, 128, 11008
    g = synth.rng(5)
    norms = [(be.alloc(H * 4).upload((1 + 0.1 * g.standard_normal(H)).astype(np.float32)),
              be.alloc(H * 4).upload((1 + 0.1 * g.standard_normal(H)).astype(np.float32)))
             for _ in model.layers]
    caches = [(be.alloc(context * kvh * hd * 4), be.alloc(context * kvh * hd * 4))
              for _ in model.layers]
    layers = []
    for lw, (an, fn) in zip(model.layers, norms):
        h = {name: handle for name, _, _, _, handle in lw}
        layers.append(RealmLayer(wq=h["wq"], wk=h["wk"], wv=h["wv"], wo=h["wo"],
                                 w_gate=h["w_gate"], w_up=h["w_up"], w_down=h["w_down"],
                                 attn_norm=an.ptr, ffn_norm=fn.ptr, hidden=H, num_heads=heads,
                                 num_kv_heads=kvh, head_dim=hd, intermediate=inter,
                                 rms_norm_eps=1e-5, rope_theta=10000.0))
    pre = context - 1
    bufs = [be.alloc(pre * H * 4), be.alloc(pre * H * 4)]
    bufs[0].upload(synth.activations(g, pre, H))

    def run(seq, pos):
        be.forward_layers_dev(layers, bufs[0].ptr, seq, pos, [c[0].ptr for c in caches],
                              [c[1].ptr for c in caches], context, bufs[1].ptr, stream=stream)

    run(pre, 0)  # prefill fills rows 0 .. context - 2 of every cache
    be.synchronize()
    # the prefill itself, replayed (every replay rewrites the same rows)
    gr = capture(be, stream, lambda: run(pre, 0))
    time_graph(be, gr, stream, 1)
    pre_ms = time_graph(be, gr, stream, 3)
    be.graph_release(gr)
    gr = capture(be, stream, lambda: run(1, pre))
    time_graph(be, gr, stream, 3)
    ms = time_graph(be, gr, stream, reps)
    be.graph_release(gr)
    for b in bufs + [x for pair in norms + caches for x in pair]:
        b.close()
    return {"ms_per_token": round(ms, 4), "tok_per_s": round(1e3 / ms, 1), "context": context,
            "prefill_ms": round(pre_ms, 3), "prefill_tok_per_s": round(pre * 1e3 / pre_ms, 1),
            "layers": len(model.layers),
            "note": "all layer steps on the device; embedding, final norm and logits excluded"}


def lora_overhead(be, stream: int, reps: int) -> dict:
    """Config 3: q_proj and v_proj (Q4_K 4096x4096) for 64 tokens, 16 adapters
    with ranks from {8,16,64}, Zipf(1.1) tenant ids, 10% without adapter.
    q and v share the input, so base and multi-LoRA products run as grouped
    calls.  Each graph holds 8 calls, timed per call: warm, all 8 on the same
    weights and adapters (resident in the 256 MB Infinity Cache); cold, on 8
    rotated copies (base + adapters), 8 x 47 MB, so weights and adapters are
    re-read from HBM; warm_per_projection: warm with one call per projection
    instead."""
    g = synth.rng(3)
    n = k = 4096
    m = 64
    copies = 8
    base_host = [synth.q4k_blocks(g, n, k) for _ in range(2)]
    ranks = [int(r) for r in g.choice([8, 16, 64], 16)]
    ad_host = [[synth.lora_adapter(g, r, k, n) for r in ranks] for _ in range(2)]
    ids = synth.adapter_ids(g, m, 16)
    x = be.alloc(m * k * 4).upload(synth.activations(g, m, k))
    d_ids = be.alloc(m * 4).upload(ids)
    y = [be.alloc(m * n * 4) for _ in range(2)]
    sets, weights, adapters = [], [], []
    for _c in range(copies):
        ws, ss = [], []
        for p in range(2):
            ws.append(be.register_weights(GGML_Q4_K, base_host[p], n, k))
            hs = [be.lora_register(a, b, r, 16.0, k, n) for (a, b), r in zip(ad_host[p], ranks)]
            adapters += hs
            ss.append(be.lora_set_create(hs))
        weights.append(ws)
        sets.append(ss)

    # q and v share their input: grouped calls (one activation prep, one
    # base launch) for the base and for the multi-LoRA product
    def base(c):
        be.matmul_group_dev(weights[c], x.ptr, m, [yy.ptr for yy in y], stream=stream)

    def lora(c):
        be.multi_lora_matmul_group_dev(weights[c], sets[c], x.ptr, m, d_ids.ptr,
                                       [yy.ptr for yy in y], stream=stream)

    # one call per projection
    def base1(c):
        for p in range(2):
            be.matmul_dev(weights[c][p], x.ptr, m, y[p].ptr, stream=stream)

    def lora1(c):
        for p in range(2):
            be.multi_lora_matmul_dev(weights[c][p], sets[c][p], x.ptr, m, d_ids.ptr, y[p].ptr,
                                     stream=stream)

    res = {}
    for mode, cs, fb, fl in (("warm", [0] * copies, base, lora),
                             ("cold", list(range(copies)), base, lora),
                             ("warm_per_projection", [0] * copies, base1, lora1)):
        gb = capture(be, stream, lambda: [fb(c) for c in cs])
        gl = capture(be, stream, lambda: [fl(c) for c in cs])
        time_graph(be, gb, stream, 5)
        time_graph(be, gl, stream, 5)
        tb = time_graph(be, gb, stream, reps) / len(cs)
        tl = time_graph(be, gl, stream, reps) / len(cs)
        be.graph_release(gb)
        be.graph_release(gl)
        res[mode] = {"base_us": round(tb * 1e3, 2), "lora_us": round(tl * 1e3, 2),
                     "overhead_pct": round((tl / tb - 1) * 100, 1)}
    distinct = sorted({int(i) for i in ids if i >= 0})
    res["distinct_adapters"] = len(distinct)
    res["adapter_bytes_per_proj"] = int(sum(2 * 2 * ranks[i] * (k + n) // 2 for i in distinct))
    for ss in sets:
        for s in ss:
            be.lora_set_release(s)
    for h in adapters:
        be.lora_release(h)
    for ws in weights:
        for w in ws:
            be.release_weights(w)
    for b in [x, d_ids] + y:
        b.close()
    return res


def prefill(be, stream: int, reps: int) -> dict:
    """Config 2: M=512, K=4096 -> N=11008, bf16 activations, f32 output."""
    g = synth.rng(2)
    m, n, k = 512, 11008, 4096
    xb = be.alloc(m * k * 2).upload(synth.activations_bf16(g, m, k))
    y = be.alloc(m * n * 4)
    out = {}
    for t, name in ((GGML_Q4_K, "q4k"), (GGML_Q8_0, "q80")):
        h = be.register_weights(t, synth.blocks(g, t, n, k), n, k)
        gr = capture(be, stream, lambda: be.matmul_dev(h, xb.ptr, m, y.ptr, stream=stream,
                                                       bf16=True))
        time_graph(be, gr, stream, 3)
        ms = time_graph(be, gr, stream, reps)
        be.graph_release(gr)
        be.release_weights(h)
        tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        out[name] = {"us": round(ms * 1e3, 1), "tflops": round(tf, 1),
                     "frac_mfma_peak": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}
    xb.close()
    y.close()
    return out


LAYER70 = [("wq", GGML_Q4_K, 8192, 8192), ("wk", GGML_Q4_K, 1024, 8192),
           ("wv", GGML_Q4_K, 1024, 8192), ("wo", GGML_Q4_K, 8192, 8192),
           ("w_gate", GGML_Q4_K, 28672, 8192), ("w_up", GGML_Q4_K, 28672, 8192),
           ("w_down", GGML_Q6_K, 8192, 28672)]


def config4(be, stream: int, reps: int) -> dict:
    """Config 4: one LLaMA-70B-shape layer (541,851,648 packed bytes, more
    than the 256 MB MALL, so every replay streams the weights from HBM).
    decode: 32 tokens (f32 activations), the base set (QKV grouped, Wo,
    gate/up grouped, W_down) against the same set with 8 rank-16 adapters on
    q/k/v/o (Zipf(1.1) ids over 8, 10% without adapter; q/k/v in one grouped
    multi-LoRA call).  prefill: 1024
    tokens, bf16 activations, the seven products one after another."""
    g = synth.rng(4)
    hs = {name: be.register_weights(t, synth.blocks(g, t, n, k), n, k)
          for name, t, n, k in LAYER70}
    dims = {name: (n, k) for name, _t, n, k in LAYER70}
    lora_on = ("wq", "wk", "wv", "wo")
    adapters, sets = [], {}
    for name in lora_on:
        n, k = dims[name]
        hl = [be.lora_register(*synth.lora_adapter(g, 16, k, n), 16, 16.0, k, n)
              for _ in range(8)]
        adapters += hl
        sets[name] = be.lora_set_create(hl)
    m_dec, m_pre = 32, 1024
    ids = synth.adapter_ids(g, m_dec, 8)
    d_ids = be.alloc(m_dec * 4).upload(ids)
    xd = {k: be.alloc(m_dec * k * 4).upload(synth.activations(g, m_dec, k))
          for k in (8192, 28672)}
    xp = {k: be.alloc(m_pre * k * 2).upload(synth.activations_bf16(g, m_pre, k))
          for k in (8192, 28672)}
    y = {name: be.alloc(m_pre * n * 4) for name, (n, _k) in dims.items()}

    def base():
        be.matmul_group_dev([hs["wq"], hs["wk"], hs["wv"]], xd[8192].ptr, m_dec,
                            [y["wq"].ptr, y["wk"].ptr, y["wv"].ptr], stream=stream)
        be.matmul_dev(hs["wo"], xd[8192].ptr, m_dec, y["wo"].ptr, stream=stream)
        be.matmul_group_dev([hs["w_gate"], hs["w_up"]], xd[8192].ptr, m_dec,
                            [y["w_gate"].ptr, y["w_up"].ptr], stream=stream)
        be.matmul_dev(hs["w_down"], xd[28672].ptr, m_dec, y["w_down"].ptr, stream=stream)

    def with_lora():
        qkv = ("wq", "wk", "wv")
        be.multi_lora_matmul_group_dev([hs[n] for n in qkv], [sets[n] for n in qkv],
                                       xd[8192].ptr, m_dec, d_ids.ptr, [y[n].ptr for n in qkv],
                                       stream=stream)
        be.multi_lora_matmul_dev(hs["wo"], sets["wo"], xd[8192].ptr, m_dec, d_ids.ptr,
                                 y["wo"].ptr, stream=stream)
        be.matmul_group_dev([hs["w_gate"], hs["w_up"]], xd[8192].ptr, m_dec,
                            [y["w_gate"].ptr, y["w_up"].ptr], stream=stream)
        be.matmul_dev(hs["w_down"], xd[28672].ptr, m_dec, y["w_down"].ptr, stream=stream)

    def pre():
        for name, _t, _n, k in LAYER70:
            be.matmul_dev(hs[name], xp[k].ptr, m_pre, y[name].ptr, stream=stream, bf16=True)

    res = {}
    wbytes = sum(weight_bytes(t, n, k) for _name, t, n, k in LAYER70)
    distinct = len({int(i) for i in ids if i >= 0})
    lbytes = distinct * sum(2 * 16 * (dims[nm][0] + dims[nm][1]) for nm in lora_on)
    act = 4 * m_dec * (8192 * 4 + 28672) + 4 * m_dec * sum(n for n, _k in dims.values())
    times = {}
    for mode, fn in (("base", base), ("lora", with_lora), ("prefill", pre)):
        gr = capture(be, stream, fn)
        time_graph(be, gr, stream, 2)
        times[mode] = time_graph(be, gr, stream, reps)
        be.graph_release(gr)
    tb, tl, tp = times["base"], times["lora"], times["prefill"]
    res["decode_m32"] = {
        "base_us": round(tb * 1e3, 1), "lora_us": round(tl * 1e3, 1),
        "lora_overhead_pct": round((tl / tb - 1) * 100, 1),
        "base_gb_per_s": round((wbytes + act) / (tb * 1e-3) / 1e9, 1),
        "lora_gb_per_s": round((wbytes + act + lbytes) / (tl * 1e-3) / 1e9, 1),
        "tok_per_s_80_layers": round(m_dec / (80 * tb * 1e-3), 1),
        "distinct_adapters": distinct, "adapter_bytes": lbytes}
    flops = 2.0 * m_pre * sum(n * k for _name, _t, n, k in LAYER70)
    res["prefill_1024"] = {"us": round(tp * 1e3, 1),
                           "tflops": round(flops / (tp * 1e-3) / 1e12, 1),
                           "frac_mfma_peak": round(flops / (tp * 1e-3) / 1e12
                                                   / MFMA_F16_PEAK_TFLOPS, 4)}
    for s in sets.values():
        be.lora_set_release(s)
    for h in adapters:
        be.lora_release(h)
    for h in hs.values():
        be.release_weights(h)
    for b in [d_ids] + list(xd.values()) + list(xp.values()) + list(y.values()):
        b.close()
    return res


def dense(be, stream: int, reps: int) -> dict:
    """The dense f32 product behind candle_matmul on device pointers:
    4096 x 4096 x 4096 (both B layouts) and a decode-shaped 32 x 4096 x 4096;
    2mnk flops against the 157.3 TFLOP/s dense f32 MFMA peak."""
    g = synth.rng(5)
    out = {}
    for name, m, k, n, tr in (("4096^3", 4096, 4096, 4096, False),
                              ("4096^3_bt", 4096, 4096, 4096, True),
                              ("32x4096x4096_bt", 32, 4096, 4096, True)):
        a = be.alloc(m * k * 4).upload(g.standard_normal((m, k), dtype=np.float32))
        b = be.alloc(k * n * 4).upload(g.standard_normal((k, n), dtype=np.float32))
        c = be.alloc(m * n * 4)
        gr = capture(be, stream, lambda: be.dense_matmul_dev(a.ptr, b.ptr, c.ptr, m, k, n,
                                                             transposed=tr, stream=stream))
        time_graph(be, gr, stream, 2)
        ms = time_graph(be, gr, stream, reps)
        be.graph_release(gr)
        tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        out[name] = {"us": round(ms * 1e3, 1), "tflops": round(tf, 1),
                     "frac_f32_mfma_peak": round(tf / 157.3, 4)}
        for d in (a, b, c):
            d.close()
    return out


CRITERION = ([("qkv_proj", 1, 6144, 2048), ("attention_out", 1, 2048, 2048),
              ("ffn_gate_up", 1, 11264, 2048), ("ffn_down", 1, 2048, 5632),
              ("lm_head", 1, 32000, 2048)]
             + [(f"batch{b}_2048", b, 2048, 2048) for b in (1, 4, 8, 16, 32)]
             + [(f"square{z}", 1, z, z) for z in (256, 512, 1024, 2048, 4096)])


def criterion_shapes(be, stream: int, reps: int) -> tuple[dict, list]:
    """The reference's own criterion workloads for the Q4_K fused kernel
    (crates/realm-compute-cpu/benches/fused_kernels.rs:96-211: the five
    transformer shapes at batch 1 including lm_head 32000 x 2048, batch sizes
    1-32 on 2048 x 2048, square matrices 256-4096), on resident weights: 20
    calls on the same weights and input per graph, as criterion's loop calls
    the same data, so the weights are cache-warm for the smaller shapes.
    Returns the GPU figures and the host data for the CPU leg."""
    g = synth.rng(11)
    out, host = {}, []
    for name, m, n, k in CRITERION:
        blocks = synth.q4k_blocks(g, n, k)
        x_host = synth.activations(g, m, k)
        h = be.register_weights(GGML_Q4_K, blocks, n, k)
        x = be.alloc(m * k * 4).upload(x_host)
        y = be.alloc(m * n * 4)
        gr = capture(be, stream, lambda: [be.matmul_dev(h, x.ptr, m, y.ptr, stream=stream)
                                          for _ in range(20)])
        time_graph(be, gr, stream, 2)
        us = time_graph(be, gr, stream, reps) / 20 * 1e3
        be.graph_release(gr)
        kern = be.last_kernel()
        out[name] = {"m": m, "n": n, "k": k, "us": round(us, 3),
                     "gb_per_s": round(alg_bytes(GGML_Q4_K, n, k, m) / (us * 1e-6) / 1e9, 1),
                     "kernel": kern}
        host.append((name, m, n, k, blocks, x_host))
        be.release_weights(h)
        x.close()
        y.close()
    return out, host


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def median_rate(fn, nbytes: int, seconds: float, trials: int = 10) -> tuple[float, int]:
    """Median GB/s over `trials` timed trials of about seconds/trials each
    (after one warm-up call); also the total number of calls."""
    fn()
    rates, calls = [], 0
    for _ in range(trials):
        t0, reps = time.perf_counter(), 0
        while reps == 0 or time.perf_counter() - t0 < seconds / trials:
            fn()
            reps += 1
        rates.append(nbytes * reps / (time.perf_counter() - t0) / 1e9)
        calls += reps
    return float(np.median(rates)), calls


def cpu_criterion(crit_host: list, gpu: dict) -> None:
    """The criterion workloads on the oracle's restatement of fused.rs (the
    function the reference's criterion benchmark times, one thread): median
    of 3 calls each, added to the GPU figures with the ratio."""
    from oracle import oracle as o  # checker/baseline only
    for name, m, n, k, blocks, x in crit_host:
        o.fused(GGML_Q4_K, blocks, x, m, n, k)
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            o.fused(GGML_Q4_K, blocks, x, m, n, k)
            ts.append(time.perf_counter() - t0)
        cpu_us = float(np.median(ts)) * 1e6
        gpu[name]["cpu_1thread_us"] = round(cpu_us, 1)
        gpu[name]["gpu_over_cpu"] = round(cpu_us / gpu[name]["us"], 1)


def cpu_baseline(seconds: float, blocks, x, gpu_y) -> tuple[dict, dict]:
    """The oracle's C restatement of realm-compute-cpu on this host's cores,
    on the timed step's own Wq (Q4_K 4096x4096) and input (batch 1):
    dequantize-row-then-dot on all cores (OpenMP, one row per iteration),
    and fused.rs semantics on one core; each the median of 10 trials within
    about `seconds`.  The oracle's output doubles as the check of the GPU's
    Wq output from the last timed step (gpu_y): relative L2 error reported."""
    from oracle import oracle as o  # checker/baseline only
    n = k = 4096
    nbytes = alg_bytes(GGML_Q4_K, n, k, 1)
    threads = len(os.sched_getaffinity(0))
    used, ref = o.fused_parallel(GGML_Q4_K, blocks, x, 1, n, k, threads)
    err = float(np.linalg.norm(gpu_y - ref) / np.linalg.norm(ref))
    par, reps = median_rate(lambda: o.fused_parallel(GGML_Q4_K, blocks, x, 1, n, k, threads),
                            nbytes, seconds)
    one, reps1 = median_rate(lambda: o.fused(GGML_Q4_K, blocks, x, 1, n, k), nbytes, seconds)
    env = {v: os.environ.get(v) for v in ("OMP_NUM_THREADS", "OMP_PROC_BIND", "OMP_PLACES")}
    base = {"value": round(par, 3), "unit": "GB/s", "cores": int(used), "kind": "port",
            "sample": f"Q4_K 4096x4096 matvec (the timed step's Wq and input), batch 1, "
                      f"dequantize row + f32 dot (CandleCpuBackend semantics), median of 10 "
                      f"trials, {reps} calls in ~{seconds:.0f}s on {used} OpenMP threads; "
                      f"oracle/realm_oracle.c",
            "cpu_model": cpu_model(), "omp_env": env,
            "gpu_check": {"output": "Wq of the last timed step", "rel_l2": err,
                          "ok": bool(err < 1e-3)}}
    single = {"value": round(one, 3), "unit": "GB/s", "cores": 1,
              "sample": f"same matvec with fused.rs semantics, median of 10 trials, "
                        f"{reps1} calls, 1 thread"}
    return base, single


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--skip-extra", action="store_true",
                    help="only the timed decode step and the roofline")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="no timing: one 256 MiB device copy (the counter reference) then "
                         "one gate/up GEMV launch per layer, for rocprofv3 --pmc runs")
    ap.add_argument("--extra-only",
                    choices=("batched", "lora", "prefill", "config4", "dense", "layer",
                             "criterion"),
                    help="run one of the extra measurements alone (for kernel profiles) and "
                         "print its result; no decode step, no JSON line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path)", file=sys.stderr)
        return 2

    from realm_amd.backend import HipGpuBackend
    be = HipGpuBackend(0)
    stream = be.stream()
    if args.extra_only == "lora":
        log(f"multi-LoRA: {lora_overhead(be, stream, 50)}")
        return 0
    if args.extra_only == "prefill":
        log(f"prefill: {prefill(be, stream, 10)}")
        return 0
    if args.extra_only == "config4":
        log(f"config4: {config4(be, stream, 10)}")
        return 0
    if args.extra_only == "dense":
        log(f"dense: {dense(be, stream, 10)}")
        return 0
    if args.extra_only == "criterion":
        log(f"criterion shapes: {criterion_shapes(be, stream, 10)[0]}")
        return 0
    log(f"registering {args.layers} LLaMA-7B layers")
    model = Model7B(be, args.layers, 16)
    if args.traffic_probe:
        nb = 256 << 20
        src, dst = be.alloc(nb), be.alloc(nb)
        be.memcpy_dtod(dst, src, nb)
        for layer in model.layers:
            model.launch_group(layer, ROOF_GROUP, 1, stream)
        be.synchronize()
        log(f"traffic probe: copy of {nb} bytes, then {len(model.layers)} x {be.last_kernel()} "
            f"({Model7B.group_bytes(ROOF_GROUP, 1)} algorithmic bytes each)")
        src.close()
        dst.close()
        model.close()
        return 0

    # ---- timed region: batch-1 decode steps replayed from one HIP graph
    m = 1
    graph = capture(be, stream, lambda: model.step(m, stream))
    for _ in range(args.warmup):
        be.graph_launch(graph, stream)
    be.synchronize()
    e0, e1 = be.event(), be.event()
    t0 = time.perf_counter()
    be.record(e0, stream)
    for _ in range(args.steps):
        be.graph_launch(graph, stream)
    be.record(e1, stream)
    be.synchronize()
    wall = (time.perf_counter() - t0) / args.steps
    ev_ms = be.elapsed_ms(e0, e1) / args.steps
    be.graph_release(graph)
    # outside the timed region: what the last step wrote for Wq (checked
    # against the oracle in the CPU-baseline leg)
    wq_out = model.y["wq"].download(np.float32, 4096)
    step_bytes = model.bytes_per_step(m)
    value = step_bytes / wall / 1e9
    log(f"decode b1: {wall * 1e3:.3f} ms/step (events {ev_ms:.3f}), {value:.1f} GB/s")

    extra = {"decode": {"b1": {"ms_per_step": round(wall * 1e3, 4),
                               "tok_per_s": round(m / wall, 1),
                               "gb_per_s": round(value, 1)}}}
    roof = decode_roofline(be, model, stream, max(5, args.steps))
    log(f"roofline: {roof['achieved']} GB/s ({roof['frac'] * 100:.1f}% of peak)")
    extra["stream_ceiling"] = stream_ceiling(be, stream, max(5, args.steps))
    log(f"stream ceiling: {extra['stream_ceiling']}")
    if args.extra_only in ("batched", "layer"):
        args.skip_extra = False
    if args.extra_only == "layer":
        log(f"full layers: {full_layers(be, model, stream, max(5, args.steps))}")
        model.close()
        return 0
    if not args.skip_extra:
        extra["full_layer_decode_7b"] = full_layers(be, model, stream, max(5, args.steps))
        log(f"full layers: {extra['full_layer_decode_7b']}")
        for mb in (4, 16):
            gr = capture(be, stream, lambda: model.step(mb, stream))
            time_graph(be, gr, stream, 2)
            ms = time_graph(be, gr, stream, max(5, args.steps // 2))
            be.graph_release(gr)
            gbs = model.bytes_per_step(mb) / (ms * 1e-3) / 1e9
            extra["decode"][f"b{mb}"] = {"ms_per_step": round(ms, 4),
                                         "tok_per_s": round(mb / (ms * 1e-3), 1),
                                         "gb_per_s": round(gbs, 1)}
            log(f"decode b{mb}: {ms:.3f} ms/step, {gbs:.1f} GB/s")
    wq_host, x_host = model.host["wq"], model.x_host[4096][:1]
    model.close()
    if args.extra_only == "batched":
        return 0
    cpu, cpu1 = None, None
    if not args.skip_extra:
        extra["multi_lora_config3"] = lora_overhead(be, stream, 50)
        log(f"multi-LoRA: {extra['multi_lora_config3']}")
        extra["prefill_config2"] = prefill(be, stream, 10)
        log(f"prefill: {extra['prefill_config2']}")
        extra["config4_70b_layer"] = config4(be, stream, 10)
        log(f"config4: {extra['config4_70b_layer']}")
        extra["dense_f32"] = dense(be, stream, 10)
        log(f"dense: {extra['dense_f32']}")
        extra["criterion_q4k"], crit_host = criterion_shapes(be, stream, 10)
        cpu_criterion(crit_host, extra["criterion_q4k"])
        log(f"criterion shapes: {extra['criterion_q4k']}")
        cpu, cpu1 = cpu_baseline(args.cpu_seconds, wq_host, x_host, wq_out)
        extra["cpu_baseline_1thread"] = cpu1
        log(f"cpu baseline: {cpu}")

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "i8dot+f32",
        "data": "synthetic (seeded, realm_amd/synth.py)",
        "config": {"workload": "config1: LLaMA-7B decoder-layer matvec set (Q4_K Wq/Wk/Wv/Wo/"
                               "W_gate/W_up, Q6_K W_down) x 32 layers, decode batch 1; "
                               "launches per layer: QKV grouped, Wo, gate/up grouped, W_down",
                   "layers": args.layers, "batch": m, "alg_bytes_per_step": step_bytes,
                   "tok_per_s": round(m / wall, 1), "hbm_frac": round(value / HBM_PEAK_GBS, 4)},
        "roofline": roof,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

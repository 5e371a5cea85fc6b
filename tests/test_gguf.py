"""GGUF images: the library's host-side parser (realm_hip_gguf_*, no GPU)
against the oracle's restatement of crates/realm-core/src/formats/gguf.rs,
and the oracle itself pinned by the reference's own header test, by byte
images assembled field by field here, and by the image writer; then, on the
GPU, tensors registered from an image by name against the oracle's matmul.
"""
import struct

import numpy as np
import pytest

import gguf_image as gi
from conftest import rel_l2
from oracle import gguf as og
from realm_amd import synth
from realm_amd.formats import GGML_Q4_K, GGML_Q6_K, GGML_Q8_0


def _model(img):
    from realm_amd.gguf import GgufModel
    return GgufModel(img)


def _code(img):
    """ErrorCode of parsing img with the library (0 if it parses)."""
    from realm_amd.backend import RealmError
    try:
        _model(img).release()
        return 0
    except RealmError as e:
        return e.code


def _ocode(img):
    try:
        og.parse(img)
        return 0
    except og.GgufError as e:
        return e.code


LLAMA_META = [
    ("general.architecture", gi.value(gi.STR, "llama")),
    ("general.name", gi.value(gi.STR, "tiny test")),
    ("llama.vocab_size", gi.value(gi.U32, 32000)),
    ("llama.embedding_length", gi.value(gi.U32, 4096)),
    ("llama.block_count", gi.value(gi.U32, 32)),
    ("llama.attention.head_count", gi.value(gi.U32, 32)),
    ("llama.attention.head_count_kv", gi.value(gi.U64, 8)),
    ("llama.feed_forward_length", gi.value(gi.I32, 11008)),
    ("llama.context_length", gi.value(gi.U32, 4096)),
    ("llama.attention.layer_norm_rms_epsilon", gi.value(gi.F32, 1e-6)),
    ("llama.rope.freq_base", gi.value(gi.F64, 500000.0)),
    ("tokenizer.ggml.tokens", gi.value(gi.ARR, ["<s>", "</s>", "é"], gi.STR)),
    ("tokenizer.ggml.scores", gi.value(gi.ARR, [0.0, -1.5, 2.25], gi.F32)),
    ("flag", gi.value(gi.BOOL, 1)),
    ("neg8", gi.value(gi.I8, -1)),
    ("big", gi.value(gi.U64, (1 << 40) + 7)),
]


def _tensors(g):
    q4 = synth.q4k_blocks(g, 8, 512).view(np.uint8).tobytes()
    q6 = synth.q6k_blocks(g, 4, 256).view(np.uint8).tobytes()
    q8 = synth.q80_blocks(g, 6, 64).view(np.uint8).tobytes()
    norm = np.arange(512, dtype=np.float32).tobytes()
    return [("blk.0.attn_q.weight", (512, 8), GGML_Q4_K, q4),
            ("blk.0.ffn_down.weight", (256, 4), GGML_Q6_K, q6),
            ("blk.0.attn_k.weight", (64, 6), GGML_Q8_0, q8),
            ("blk.0.attn_norm.weight", (512,), 0, norm)]


# ------------------------------------------------------- oracle pinned

def test_oracle_reference_header_test():
    """gguf.rs:487-503 (test_gguf_magic): v3, no tensors, no metadata."""
    img = struct.pack("<IIQQ", 0x46554747, 3, 0, 0)
    m = og.parse(img)
    assert m["version"] == 3 and m["tensor_count"] == 0 and m["tensors"] == []
    assert m["data_offset"] == 32  # 24 header bytes rounded up to 32


def test_oracle_hand_assembled_image():
    """Every field written byte by byte here, independently of the writer."""
    img = b"GGUF" + (2).to_bytes(4, "little") + (1).to_bytes(8, "little") + \
        (2).to_bytes(8, "little")
    img += (3).to_bytes(8, "little") + b"a.b" + (4).to_bytes(4, "little") + \
        (7).to_bytes(4, "little")                              # u32 7
    img += (1).to_bytes(8, "little") + b"s" + (9).to_bytes(4, "little") + \
        (3).to_bytes(4, "little") + (2).to_bytes(8, "little") + \
        (-2).to_bytes(2, "little", signed=True) + (5).to_bytes(2, "little")  # i16 [-2, 5]
    img += (2).to_bytes(8, "little") + b"wq" + (2).to_bytes(4, "little") + \
        (256).to_bytes(8, "little") + (3).to_bytes(8, "little") + \
        (12).to_bytes(4, "little") + (64).to_bytes(8, "little")
    m = og.parse(img)
    assert m["version"] == 2 and m["kv_count"] == 2
    assert m["metadata"]["a.b"] == (4, 7)
    assert m["metadata"]["s"] == (9, [(3, -2), (3, 5)])
    assert m["tensors"] == [("wq", (256, 3), 12, 64)]
    assert m["data_offset"] == (len(img) + 31) // 32 * 32


def test_oracle_reads_back_the_writer():
    g = synth.rng(7)
    ts = _tensors(g)
    img = gi.image(LLAMA_META, ts)
    m = og.parse(img)
    assert [t[0] for t in m["tensors"]] == [t[0] for t in ts]
    for (name, dims, ty, off), (_, wdims, wty, payload) in zip(m["tensors"], ts):
        assert dims == wdims and ty == wty
        a = m["data_offset"] + off
        assert img[a:a + len(payload)] == payload
    assert og.as_u32(m["metadata"]["neg8"]) == 0xFFFFFFFF
    assert og.as_u32(m["metadata"]["big"]) == 7
    assert og.as_u32(m["metadata"]["general.name"]) is None


# ------------------------------------------------- library vs oracle

def test_parse_matches_oracle():
    g = synth.rng(8)
    img = gi.image(LLAMA_META, _tensors(g))
    ref = og.parse(img)
    m = _model(img)
    try:
        assert (m.version, m.tensor_count, m.metadata_kv_count, m.data_offset) == \
            (ref["version"], ref["tensor_count"], ref["kv_count"], ref["data_offset"])
        sizes = {GGML_Q4_K: 144 / 256, GGML_Q6_K: 210 / 256, GGML_Q8_0: 34 / 32, 0: 4}
        for i, (name, dims, ty, off) in enumerate(ref["tensors"]):
            t = m.tensor(i)
            assert (t.name, t.ggml_type, t.dims) == (name, ty, dims)
            assert t.offset == ref["data_offset"] + off
            assert t.nbytes == int(np.prod(dims) * sizes[ty])
            assert m.find(name) == i
        for key, v in ref["metadata"].items():
            assert m.meta_u32(key) == og.as_u32(v), key
            assert m.meta_str(key) == (v[1] if v[0] == 8 else None), key
        assert m.extract_config() == pytest.approx(og.extract_config(ref))
    finally:
        m.release()


@pytest.mark.parametrize("case", ["full", "empty", "fallback", "wrong_type", "other_arch"])
def test_extract_config_matches_oracle(case):
    """Keys, fallback keys and defaults of extract_config: with every key, with
    none (defaults), with only the second keys, with a first key of the wrong
    type (no fallback then: or_else only looks at presence), and an
    architecture whose keys are missing."""
    meta = {
        "full": LLAMA_META,
        "empty": [],
        "fallback": [("general.architecture", gi.value(gi.STR, "qwen")),
                     ("vocab_size", gi.value(gi.U16, 1000)),
                     ("qwen.hidden_size", gi.value(gi.U32, 896)),
                     ("qwen.num_layers", gi.value(gi.I64, 24)),
                     ("qwen.num_heads", gi.value(gi.U8, 14)),
                     ("qwen.num_kv_heads", gi.value(gi.U8, 2)),
                     ("qwen.intermediate_size", gi.value(gi.U32, 4864)),
                     ("qwen.max_seq_len", gi.value(gi.U32, 32768)),
                     ("rms_norm_eps", gi.value(gi.F64, 1e-6)),
                     ("rope_theta", gi.value(gi.F32, 1e6))],
        "wrong_type": [("general.architecture", gi.value(gi.STR, "llama")),
                       ("llama.embedding_length", gi.value(gi.STR, "4096")),
                       ("llama.hidden_size", gi.value(gi.U32, 4096)),
                       ("llama.rope.freq_base", gi.value(gi.U32, 7)),
                       ("rope_theta", gi.value(gi.F32, 3.0))],
        "other_arch": [("general.architecture", gi.value(gi.STR, "phi3")),
                       ("llama.block_count", gi.value(gi.U32, 80))],
    }[case]
    img = gi.image(meta)
    m = _model(img)
    try:
        got, ref = m.extract_config(), og.extract_config(og.parse(img))
    finally:
        m.release()
    assert got == pytest.approx(ref)
    if case == "empty":
        assert got["hidden_size"] == 2048 and got["num_kv_heads"] == 4
    if case == "wrong_type":
        assert got["hidden_size"] == 2048 and got["rope_theta"] == 10000.0


def test_error_cases_match_oracle():
    base = gi.image(LLAMA_META, _tensors(synth.rng(9)))
    cases = {
        "magic": b"GGUX" + base[4:],
        "version1": base[:4] + struct.pack("<I", 1) + base[8:],
        "version4": base[:4] + struct.pack("<I", 4) + base[8:],
        "value_type": gi.image([("k", struct.pack("<I", 13) + b"\0" * 8)]),
        "nested_array": gi.image([("k", struct.pack("<IIQ", 9, 9, 1) + b"\0" * 12)]),
        "empty_nested_array": gi.image([("k", struct.pack("<IIQ", 9, 9, 0))]),
        "utf8": gi.image([("k", gi.value(gi.STR, b"\xff\xfe"))]),
        "utf8_surrogate": gi.image([("k", gi.value(gi.STR, b"\xed\xa0\x80"))]),
        "zero_dim": gi.image([], [("t", (256, 0), GGML_Q4_K, b"")]),
        "empty_shape": gi.image([], [("t", (), GGML_Q4_K, b"")]),
    }
    expect = {"magic": 4, "version1": 4, "version4": 4, "value_type": 4, "nested_array": 4,
              "empty_nested_array": 0, "utf8": 4, "utf8_surrogate": 4, "zero_dim": 3,
              "empty_shape": 3}
    for name, img in cases.items():
        assert _ocode(img) == expect[name], name
        assert _code(img) == expect[name], name


def test_every_truncation_is_an_io_error():
    """Any prefix that ends inside the header (metadata or tensor table) is
    read_exact past the end: Error::Io (ErrorCode 7), in the oracle and the
    library alike; the header's full length parses."""
    img = gi.image(LLAMA_META[:6], _tensors(synth.rng(10))[:2])
    hdr_end = og.parse(img)["data_offset"]
    table_end = min(n for n in range(hdr_end + 1) if _ocode(img[:n]) != 7)
    for n in range(table_end):
        assert _ocode(img[:n]) == 7 and _code(img[:n]) == 7, n
    assert _code(img[:table_end]) == 0


def test_alignment_key_and_repeated_names():
    """general.alignment moves the data section (the reference keeps 32: the
    library follows the format here), and a repeated tensor name finds the
    last one (as the name-keyed tensor map keeps it)."""
    g = synth.rng(11)
    q4 = synth.q4k_blocks(g, 2, 256).view(np.uint8).tobytes()
    img = gi.image([("general.alignment", gi.value(gi.U32, 64))],
                   [("w", (256, 2), GGML_Q4_K, q4), ("w", (256, 2), GGML_Q4_K, q4)],
                   alignment=64)
    m = _model(img)
    try:
        assert m.data_offset % 64 == 0 and m.data_offset >= og.parse(img)["data_offset"]
        assert m.find("w") == 1
        t = m.tensor(1)
        assert img[t.offset:t.offset + t.nbytes] == q4
    finally:
        m.release()
    bad = gi.image([("general.alignment", gi.value(gi.U32, 48))])
    assert _code(bad) == 4


# ------------------------------------------------------------- GPU

@pytest.mark.gpu
def test_registered_tensors_by_name(backend, oracle):
    """Every 2-D Q4_K / Q6_K / Q8_0 tensor registered once from the image;
    products through the handle found by name against the oracle's fused
    matmul on the bytes at the oracle parser's offsets; the 1-D f32 tensor
    is listed but not a weight; a second register call adds nothing."""
    from realm_amd.backend import BackendError
    g = synth.rng(12)
    ts = _tensors(g)
    img = gi.image(LLAMA_META, ts)
    ref = og.parse(img)
    m = _model(img)
    try:
        assert m.register() == 3
        assert m.register() == 0
        for name, dims, ty, off in ref["tensors"]:
            if ty == 0:
                with pytest.raises(BackendError):
                    m.weight(name)
                continue
            h, n, k = m.weight(name)
            assert (n, k) == (dims[1], dims[0])
            a = ref["data_offset"] + off
            raw = np.frombuffer(img, np.uint8, count=int(n * k * {12: 144 / 256, 14: 210 / 256,
                                                                   8: 34 / 32}[ty]), offset=a)
            for mm in (1, 3, 40):
                x = synth.activations(g, mm, k)
                got = backend.weights_matmul(h, x)
                blocks = raw.view({12: synth.q4k_blocks(g, 1, 256).dtype,
                                   14: synth.q6k_blocks(g, 1, 256).dtype,
                                   8: synth.q80_blocks(g, 1, 32).dtype}[ty])
                rc, want = oracle.candle_fused(ty, blocks, x, mm, n, k)
                assert rc == 0 and rel_l2(got, want.reshape(mm, n)) < 1e-3, (name, mm)
    finally:
        m.release()


@pytest.mark.gpu
def test_registered_block32_tensors(backend, oracle):
    """A hand-assembled image with Q4_0 (18-byte blocks) and Q5_1 (24-byte
    blocks) tensors, the byte sizes GGUF gives them: the library's and the
    oracle parser's tensor tables agree on types and offsets, both register
    as resident weights, and their products agree with the oracle's fused
    matmul on the bytes at those offsets."""
    g = np.random.default_rng(13)
    specs = [("blk.0.attn_q.weight", 2, 18, 96, 256), ("blk.0.ffn_up.weight", 7, 24, 64, 512)]
    ts = []
    for name, ty, bb, n, k in specs:
        raw = g.integers(0, 256, (n * k // 32, bb), dtype=np.uint8)
        sc = (np.abs(g.standard_normal(n * k // 32)) * 1e-2).astype(np.float16).view(np.uint16)
        raw[:, 0], raw[:, 1] = sc & 0xFF, sc >> 8
        if ty == 7:  # Q5_1 delta
            dl = (g.standard_normal(n * k // 32) * 1e-3).astype(np.float16).view(np.uint16)
            raw[:, 2], raw[:, 3] = dl & 0xFF, dl >> 8
        ts.append((name, [k, n], ty, raw.tobytes()))
    img = gi.image(LLAMA_META, ts)
    ref = og.parse(img)
    m = _model(img)
    try:
        got_table = [(t.name, t.ggml_type, t.offset, t.nbytes) for t in m.tensors()]
        assert got_table == [(nm, ty, ref["data_offset"] + off, n * k // 32 * bb)
                             for (nm, _d, ty, off), (_, _, bb, n, k) in zip(ref["tensors"], specs)]
        assert m.register() == 2
        for (name, ty, bb, n, k), (_, _, _, off) in zip(specs, ref["tensors"]):
            h, nn, kk = m.weight(name)
            assert (nn, kk) == (n, k)
            a = ref["data_offset"] + off
            raw = np.frombuffer(img, np.uint8, count=n * k // 32 * bb, offset=a)
            for mm in (1, 6):
                x = g.standard_normal((mm, k)).astype(np.float32)
                rc, want = oracle.candle_fused(ty, raw, x, mm, n, k)
                assert rc == 0 and rel_l2(backend.weights_matmul(h, x), want.reshape(mm, n)) < 1e-3
    finally:
        m.release()

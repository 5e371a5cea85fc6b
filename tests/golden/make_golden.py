"""Write tests/golden/kat.npz: known-answer vectors for the quantized path.

Inputs are the reference's own test inputs; expected outputs are written down
in closed form here (never produced by the oracle or the HIP library), so the
fixtures check both.  Sources:

  q4k_kat    crates/realm-core/src/quant.rs:975-1003  (d=1, dmin=0.5, scales
             0x11, qs 0x50).  get_scale_min_k4 gives sc=m=17 for sub-blocks
             0..3 and sc=m=1 for 4..7; low nibble 0, high nibble 5, so the
             four 64-groups are (-8.5 x32, 76.5 x32, -8.5, 76.5, -0.5, 4.5,
             -0.5, 4.5) per 32 elements.
  q6k_kat    quant.rs:1005-1040 (scales 1, d=1, ql[0]=0x10, everything else
             0): every 6-bit value is 0 -> -32, except the high nibble of
             ql[0], which feeds element 64 -> 1 - 32 = -31.
  q8_kat     quant.rs:962-973 (scale 0.25, quants 10) -> 2.5.
  q4k_pos    one-hot nibble probes: low nibble of qs[32g+j] -> element 64g+j,
             high nibble -> 64g+32+j (the ggml Q4_K layout), with d=1,
             dmin=0 and every sub-block scale 1, so the element equals 15.
  q6k_pos    one-hot probes of the Q6_K layout: ql[64h+l] low/high nibble ->
             elements 128h+l / 128h+l+64, ql[64h+l+32] low/high -> +32 / +96,
             with the 2 high bits from qh[32h+l] bits (0-1, 2-3, 4-5, 6-7);
             value 63 - 32 = 31 at the probe, -32 elsewhere.
  dense      crates/realm-compute-cpu/src/gemm.rs:197-226 ([22,28,49,64],
             [7,10,15,22]) and crates/realm-compute-gpu/src/
             candle_backend.rs:1258-1276 ([19,22,43,50]).
  lora       crates/realm-runtime/src/lora.rs:227-260 (r=2, alpha=4, A=B=0.5,
             base 1 -> 1 + 2*(0.5*0.5+0.5*0.5) = 2.0) and
             crates/realm-runtime/tests/integration_frameworks.rs:9-34 (r=4,
             alpha=8, A=0.1, B=0.2 -> 1 + 2*sum of four f32 products).
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
F16 = lambda v: int(np.float16(v).view(np.uint16))  # noqa: E731


def q4k_block(d, dmin, scales, qs):
    b = bytearray()
    b += int(d).to_bytes(2, "little") + int(dmin).to_bytes(2, "little")
    b += bytes(scales) + bytes(qs)
    assert len(b) == 144
    return np.frombuffer(bytes(b), np.uint8)


def q6k_block(ql, qh, scales, d):
    b = bytes(ql) + bytes(qh) + np.asarray(scales, np.int8).tobytes() + int(d).to_bytes(2, "little")
    assert len(b) == 210
    return np.frombuffer(b, np.uint8)


def main():
    out = {}
    # --- Q4_K KAT
    out["q4k_kat_block"] = q4k_block(F16(1.0), F16(0.5), [0x11] * 12, [0x50] * 128)
    per32 = [-8.5, 76.5, -8.5, 76.5, -0.5, 4.5, -0.5, 4.5]
    out["q4k_kat_expected"] = np.repeat(np.array(per32, np.float32), 32)
    # --- Q6_K KAT
    ql = [0] * 128
    ql[0] = 0x10
    out["q6k_kat_block"] = q6k_block(ql, [0] * 64, [1] * 16, F16(1.0))
    e = np.full(256, -32.0, np.float32)
    e[64] = -31.0
    out["q6k_kat_expected"] = e
    # --- Q8_0 KAT
    out["q8_kat_block"] = np.frombuffer(F16(0.25).to_bytes(2, "little") + bytes([10] * 32), np.uint8)
    out["q8_kat_expected"] = np.full(32, 2.5, np.float32)
    # --- Q4_K position probes: 256 blocks, one per (byte, nibble)
    scales = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]  # sc=1, m=0 for all 8 sub-blocks
    blocks, idx = [], []
    for byte in range(128):
        for hi in range(2):
            qs = [0] * 128
            qs[byte] = 0xF0 if hi else 0x0F
            blocks.append(q4k_block(F16(1.0), F16(0.0), scales, qs))
            g, j = divmod(byte, 32)
            idx.append(64 * g + 32 * hi + j)
    out["q4k_pos_blocks"] = np.concatenate(blocks)
    out["q4k_pos_index"] = np.array(idx, np.int32)
    # --- Q6_K position probes: 256 blocks, one per element
    blocks, idx = [], []
    for h in range(2):
        for l in range(32):
            for t in range(4):
                ql = [0] * 128
                qh = [0] * 64
                ql_i = 64 * h + l + (32 if t & 1 else 0)
                ql[ql_i] = 0xF0 if t & 2 else 0x0F
                qh[32 * h + l] = 3 << (2 * t)
                blocks.append(q6k_block(ql, qh, [1] * 16, F16(1.0)))
                idx.append(128 * h + l + 32 * t)
    out["q6k_pos_blocks"] = np.concatenate(blocks)
    out["q6k_pos_index"] = np.array(idx, np.int32)
    # --- dense KATs: (a, b, m, k, n, transposed, expected)
    out["dense_a1"] = np.array([1, 2, 3, 4, 5, 6], np.float32)
    out["dense_b1"] = np.array([1, 2, 3, 4, 5, 6], np.float32)
    out["dense_e1"] = np.array([22, 28, 49, 64], np.float32)  # m=2,k=3,n=2
    out["dense_a2"] = np.array([1, 2, 3, 4], np.float32)
    out["dense_bt2"] = np.array([1, 3, 2, 4], np.float32)
    out["dense_e2"] = np.array([7, 10, 15, 22], np.float32)  # B^T form, m=k=n=2
    out["dense_a3"] = np.array([1, 2, 3, 4], np.float32)
    out["dense_b3"] = np.array([5, 6, 7, 8], np.float32)
    out["dense_e3"] = np.array([19, 22, 43, 50], np.float32)
    # --- LoRA KATs
    out["lora1_expected"] = np.full(16, 2.0, np.float32)
    p = np.float32(0.2) * np.float32(0.1)
    s = np.float32(0)
    for _ in range(4):
        s = np.float32(s + p)
    out["lora2_expected"] = np.full(16, np.float32(1) + np.float32(s * np.float32(2.0)), np.float32)
    np.savez(os.path.join(HERE, "kat.npz"), **out)
    print("wrote", os.path.join(HERE, "kat.npz"), sorted(out))


if __name__ == "__main__":
    main()

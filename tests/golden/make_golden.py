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
  q5k_kat    quant.rs:1043-1075 (the reference's own 178-byte Q5_K: scales 1,
             d=1, ql[0]=0x10, the rest 0): element 0 is the byte 0x10 = 16;
             every other element of 0..127 is 0, and 128..255 are never
             written (ql holds 128 bytes) -> 0.
  q8k_kat    quant.rs:1077-1109 (292-byte Q8_K: d=1, dmin=0, quants[0]=10,
             scales[0]=0x11): groups 0 and 1 have scale 1, the rest 0, and
             only quants[0] is non-zero -> 10 at element 0, 0 elsewhere.
  q2k_pos /  one-hot probes of the reference's Q2_K (116 B) and Q3_K (196 B):
  q3k_pos    element i takes its two low bits from qs[i/4] at bit 2(i%4)
             and its third bit from qh[i/8] at bit i%8 (quant.rs:565-575,
             614-624); the probe sets all three for element i only, so q is
             7 - 2 = 5 (Q2_K) or 7 - 4 = 3 (Q3_K) there and -2 / -4 elsewhere.
             Q2_K scales 0x11 (every group scale 1); Q3_K scales 0xFF, whose
             group scales are (0xFF >> 2(l%4)) & 63 = 63, 63, 15, 3 for
             l%4 = 0..3 (groups of 8).  d=1, dmin=0.
  q2k_scale  Q2_K scale nibbles: scales[j] = 2j | (2j+1) << 4 gives group l
             (16 elements) the scale l; every q is (1 | 0) - 2 = -1, so
             element i is -(i // 16).
  q3k_scale  Q3_K scales all 0xE4: group scales 0x24 = 36, 0x39 = 57,
             0xE4 >> 4 = 14, 0xE4 >> 6 = 3 for l%4 = 0..3; every q is 1 - 4 =
             -3 -> -3 x those, eight elements per group.
  q5k_pos    Q5_K probes: ql[i] = 0x0F for one i < 128 -> 15 there (scales 1,
             d=1), 0 elsewhere; ql[i] = 0x80 -> int8 -128; qh[j] = 0x0F sets
             the fifth bit of elements 16(j//2) + 8(j%2) + 0..3 (byte 0xF0 as
             int8: -16), qh[j] = 0xF0 of elements 16(j//2) + 8(j%2) + 4..7;
             qh[16..31] feed nothing.
  q8k_scale  Q8_K: scales[j] = 0x21 for j < 16 and 0xFF beyond (unused:
             groups read scales[l/2] for l < 32); quants 1, d=1, dmin=0.5 ->
             group scale 1 or 2 by group parity: 1.5 and 2.5 in runs of 8.
  q5_0_qh /  the reference's own Q5_0 / Q5_1 high-bit map (quant.rs:283-350),
  q5_1_qh    written out by hand: in each qh byte j, Q5_0 feeds elements
             8j + (0,1) from bit 0, (4,5) from bit 2, (2,3) from bit 4, (6,7)
             from bit 6 (bits 1, 3, 5, 7 unused); Q5_1 feeds 8j + (0,1,4,5)
             from bit 0 and (2,3,6,7) from bit 4.  With ql all 0 and scale 1,
             a fed element is 16 - 16 = 0 and every other one -16.
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
    # --- the reference's own Q5_K / Q8_K / Q2_K / Q3_K layouts
    def q5k_block(ql, qh, scales, d):
        b = bytes(ql) + bytes(qh) + np.asarray(scales, np.int8).tobytes() + int(d).to_bytes(2, "little")
        assert len(b) == 178
        return np.frombuffer(b, np.uint8)

    def q8k_block(quants, scales, d, dmin):
        b = np.asarray(quants, np.int8).tobytes() + bytes(scales) + int(d).to_bytes(2, "little")
        b += int(dmin).to_bytes(2, "little")
        assert len(b) == 292
        return np.frombuffer(b, np.uint8)

    def q23k_block(nsc, scales, qh, qs, d, dmin):
        b = int(d).to_bytes(2, "little") + int(dmin).to_bytes(2, "little")
        b += bytes(scales) + bytes(qh) + bytes(qs)
        assert len(b) == (116 if nsc == 16 else 196)
        return np.frombuffer(b, np.uint8)

    ql = [0] * 128
    ql[0] = 0x10
    out["q5k_kat_block"] = q5k_block(ql, [0] * 32, [1] * 16, F16(1.0))
    e = np.zeros(256, np.float32)
    e[0] = 16.0
    out["q5k_kat_expected"] = e
    qu = [0] * 256
    qu[0] = 10
    sc = [0] * 32
    sc[0] = 0x11
    out["q8k_kat_block"] = q8k_block(qu, sc, F16(1.0), F16(0.0))
    e = np.zeros(256, np.float32)
    e[0] = 10.0
    out["q8k_kat_expected"] = e
    # Q2_K / Q3_K one-hot probes, one block per element
    q3_group_scale = [63, 63, 15, 3]  # (0xFF >> 2(l%4)) & 63
    for name, nsc, scales, hot, cold in (("q2k", 16, [0x11] * 16, 5.0, -2.0),
                                         ("q3k", 32, [0xFF] * 32, 3.0, -4.0)):
        nqs = 64 if nsc == 16 else 128
        blocks, exp = [], []
        for i in range(256):
            qs = [0] * nqs
            qh = [0] * 32
            qs[i // 4] = 3 << (2 * (i % 4))
            qh[i // 8] = 1 << (i % 8)
            blocks.append(q23k_block(nsc, scales, qh, qs, F16(1.0), F16(0.0)))
            row = np.full(256, cold, np.float32)
            row[i] = hot
            if name == "q3k":
                row *= np.array([q3_group_scale[(j // 8) % 4] for j in range(256)], np.float32)
            exp.append(row)
        out[f"{name}_pos_blocks"] = np.concatenate(blocks)
        out[f"{name}_pos_expected"] = np.concatenate(exp)
    # scale maps: every q-bit pattern (qs 1, qh 0) in every element
    qs1 = [0x55] * 64  # 2-bit fields all 1
    out["q2k_scale_block"] = q23k_block(16, [(2 * j) | ((2 * j + 1) << 4) for j in range(8)] + [0] * 8,
                                        [0] * 32, qs1, F16(1.0), F16(0.0))
    out["q2k_scale_expected"] = -np.repeat(np.arange(16, dtype=np.float32), 16)
    out["q3k_scale_block"] = q23k_block(32, [0xE4] * 32, [0] * 32, [0x55] * 128, F16(1.0), F16(0.0))
    out["q3k_scale_expected"] = np.tile(np.repeat(np.array([36, 57, 14, 3], np.float32), 8), 8) * -3
    # Q5_K probes
    blocks, exp = [], []
    for i in range(128):
        for byte, val in ((0x0F, 15.0), (0x80, -128.0)):
            ql = [0] * 128
            ql[i] = byte
            blocks.append(q5k_block(ql, [0] * 32, [1] * 16, F16(1.0)))
            row = np.zeros(256, np.float32)
            row[i] = val
            exp.append(row)
    for j in range(32):
        for byte in (0x0F, 0xF0):
            qh = [0] * 32
            qh[j] = byte
            blocks.append(q5k_block([0] * 128, qh, [1] * 16, F16(1.0)))
            row = np.zeros(256, np.float32)
            if j < 16:
                first = 16 * (j // 2) + 8 * (j % 2) + (0 if byte == 0x0F else 4)
                row[first:first + 4] = -16.0
            exp.append(row)
    out["q5k_pos_blocks"] = np.concatenate(blocks)
    out["q5k_pos_expected"] = np.concatenate(exp)
    # Q8_K scale map
    out["q8k_scale_block"] = q8k_block([1] * 256, [0x21] * 16 + [0xFF] * 16, F16(1.0), F16(0.5))
    out["q8k_scale_expected"] = np.tile(np.repeat(np.array([1.5, 2.5], np.float32), 8), 16)
    # Q5_0 / Q5_1 high-bit tables (hand-written from quant.rs:283-350)
    Q50_BITS = {0: (0, 1), 2: (4, 5), 4: (2, 3), 6: (6, 7)}
    Q51_BITS = {0: (0, 1, 4, 5), 4: (2, 3, 6, 7)}
    for name, bb, table in (("q5_0", 22, Q50_BITS), ("q5_1", 24, Q51_BITS)):
        blocks, exp = [], []
        for j in range(4):
            for bit in range(8):
                b = bytearray(bb)
                b[0:2] = F16(1.0).to_bytes(2, "little")
                qh_off = 2 if bb == 22 else 4  # Q5_1: scale, delta (0), qh
                b[qh_off + j] = 1 << bit
                blocks.append(np.frombuffer(bytes(b), np.uint8))
                row = np.full(32, -16.0, np.float32)
                for el in table.get(bit, ()):
                    row[8 * j + el] = 0.0
                exp.append(row)
        out[f"{name}_qh_blocks"] = np.concatenate(blocks)
        out[f"{name}_qh_expected"] = np.concatenate(exp)
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

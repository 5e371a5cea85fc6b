// Dequantization (bit-exact with the reference CPU dequantizer) and the
// repack of reference-layout blocks into the device layout described in
// common.h.  Both read the reference's packed blocks as raw bytes.
#include "common.h"

using namespace realm;

// The reference never contracts `d1 * x - m1` into an FMA
// (crates/realm-core/src/quant.rs:175,182); neither may we.  The pragma is
// scoped to each dequant kernel body: every other kernel of the code object
// (one translation unit) keeps FMA contraction.

// quant.rs:127-187.  One thread per qs byte: 128 threads per block, two
// outputs each (low nibble -> k = 64g + j, high nibble -> k = 64g + 32 + j).
extern "C" __global__ __launch_bounds__(256) void realm_dequant_q4k(
    const uint8_t *__restrict__ raw, float *__restrict__ out, long long nblocks)
{
#pragma clang fp contract(off)
    long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long b = gid >> 7;
    if (b >= nblocks)
        return;
    int byte = (int)(gid & 127);
    int g = byte >> 5, j = byte & 31;
    const uint8_t *blk = raw + b * Q4K_BLOCK_BYTES;
    uint32_t dbits = blk[0] | (blk[1] << 8);
    uint32_t mbits = blk[2] | (blk[3] << 8);
    const uint8_t *s = blk + 4;
    uint32_t s0 = s[0] | (s[1] << 8) | (s[2] << 16) | ((uint32_t)s[3] << 24);
    uint32_t s1 = s[4] | (s[5] << 8) | (s[6] << 16) | ((uint32_t)s[7] << 24);
    uint32_t s2 = s[8] | (s[9] << 8) | (s[10] << 16) | ((uint32_t)s[11] << 24);
    uint32_t sc_lo, m_lo, sc_hi, m_hi;
    q4k_scale_min_pair(s0, s1, s2, g, sc_lo, m_lo, sc_hi, m_hi);
    float d = f16_bits_to_f32(dbits);
    float dmin = f16_bits_to_f32(mbits);
    float d1 = d * (float)sc_lo, m1 = dmin * (float)m_lo;
    float d2 = d * (float)sc_hi, m2 = dmin * (float)m_hi;
    uint32_t q = blk[16 + byte];
    float *y = out + b * QK_K + 64 * g;
    y[j] = d1 * (float)(q & 0xF) - m1;
    y[32 + j] = d2 * (float)(q >> 4) - m2;
}

// quant.rs:393-451.  One thread per (block, half h, l): four outputs
// y[128h + l + 32t] = (d * sc[8h + l/16 + 2t]) * q_t.
extern "C" __global__ __launch_bounds__(256) void realm_dequant_q6k(
    const uint8_t *__restrict__ raw, float *__restrict__ out, long long nblocks)
{
#pragma clang fp contract(off)
    long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long b = gid >> 6;
    if (b >= nblocks)
        return;
    int h = (int)((gid >> 5) & 1), l = (int)(gid & 31);
    const uint8_t *blk = raw + b * Q6K_BLOCK_BYTES;
    const uint8_t *ql = blk + 64 * h;
    const uint8_t *qh = blk + 128 + 32 * h;
    const int8_t *sc = reinterpret_cast<const int8_t *>(blk + 192) + 8 * h;
    float d = f16_bits_to_f32(blk[208] | (blk[209] << 8));
    int is = l >> 4;
    uint32_t a = ql[l], bq = ql[l + 32], hb = qh[l];
    int q1 = (int)((a & 0xF) | ((hb & 3) << 4)) - 32;
    int q2 = (int)((bq & 0xF) | (((hb >> 2) & 3) << 4)) - 32;
    int q3 = (int)((a >> 4) | (((hb >> 4) & 3) << 4)) - 32;
    int q4 = (int)((bq >> 4) | (((hb >> 6) & 3) << 4)) - 32;
    float *y = out + b * QK_K + 128 * h + l;
    y[0] = d * (float)sc[is] * (float)q1;
    y[32] = d * (float)sc[is + 2] * (float)q2;
    y[64] = d * (float)sc[is + 4] * (float)q3;
    y[96] = d * (float)sc[is + 6] * (float)q4;
}

// quant.rs:371-387: y = q * d, one thread per element.
extern "C" __global__ __launch_bounds__(256) void realm_dequant_q80(
    const uint8_t *__restrict__ raw, float *__restrict__ out, long long nblocks)
{
#pragma clang fp contract(off)
    long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long b = gid >> 5;
    if (b >= nblocks)
        return;
    int i = (int)(gid & 31);
    const uint8_t *blk = raw + b * Q80_BLOCK_BYTES;
    float d = f16_bits_to_f32(blk[0] | (blk[1] << 8));
    out[gid] = (float)(int8_t)blk[2 + i] * d;
}

// ------------------------------------------------------------------ repack

// Q4_K: a 144-byte block is nine 16-byte pieces (the raw buffer is 256-byte
// aligned and 144 = 9*16): piece 0 -> hdr (scale/min pairs re-packed per
// group, see common.h), piece 1 + 2g + h -> plane h of unit 4*kb + g of the
// block's row, high nibbles XOR 8.
extern "C" __global__ __launch_bounds__(256) void realm_repack_q4k(
    const uint8_t *__restrict__ raw, uint8_t *__restrict__ hdr, uint8_t *__restrict__ qs,
    long long nblocks, int blocks_per_row)
{
    long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long b = gid / 9;
    if (b >= nblocks)
        return;
    int piece = (int)(gid - b * 9);
    uint4 v = ldg16(raw + b * Q4K_BLOCK_BYTES + 16 * piece);
    if (piece == 0) {
        uint64_t f0 = 0, f1 = 0; // 96-bit field, low and high parts
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            uint32_t sl, ml, sh, mh;
            q4k_scale_min_pair(v.y, v.z, v.w, g, sl, ml, sh, mh);
            const uint64_t pair = sl | (ml << 6) | (sh << 12) | (mh << 18);
            const int at = 24 * g; // 0, 24, 48, 72
            if (at < 64)
                f0 |= pair << at;
            if (at + 24 > 64)
                f1 |= at < 64 ? pair >> (64 - at) : pair << (at - 64);
        }
        v.y = (uint32_t)f0;
        v.z = (uint32_t)(f0 >> 32);
        v.w = (uint32_t)f1;
        *reinterpret_cast<uint4 *>(hdr + b * 16) = v;
        return;
    }
    long long row = b / blocks_per_row;
    int kb = (int)(b - row * blocks_per_row);
    int g = (piece - 1) >> 1, h = (piece - 1) & 1;
    long long U = 4LL * blocks_per_row;
    v.x ^= 0x80808080u;
    v.y ^= 0x80808080u;
    v.z ^= 0x80808080u;
    v.w ^= 0x80808080u;
    *reinterpret_cast<uint4 *>(qs + row * (U * 32) + h * (U * 16) + (4 * kb + g) * 16) = v;
}

// Q6_K: 64 threads per block.  Thread t writes quant bytes t, t+64, t+128 of
// the block's four 48-byte units (unit v: ql_a, ql_b, qh -> planes 0, 1, 2),
// threads 0..15 the regrouped scales and thread 0 the f16 scale.
extern "C" __global__ __launch_bounds__(256) void realm_repack_q6k(
    const uint8_t *__restrict__ raw, uint8_t *__restrict__ dq, int8_t *__restrict__ scq,
    uint8_t *__restrict__ qq, long long nblocks, int blocks_per_row)
{
    long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long b = gid >> 6;
    if (b >= nblocks)
        return;
    int t = (int)(gid & 63);
    const uint8_t *blk = raw + b * Q6K_BLOCK_BYTES;
    long long row = b / blocks_per_row;
    int kb = (int)(b - row * blocks_per_row);
    long long U = 4LL * blocks_per_row;
    for (int o = t; o < 192; o += 64) {
        int v = o / 48, r = o - 48 * v; // unit v, byte r of its 48
        int h = v >> 1, is = v & 1;
        int plane = r >> 4, j = r & 15;
        uint8_t val;
        if (plane == 0)
            val = blk[64 * h + 16 * is + j]; // ql_a
        else if (plane == 1)
            val = blk[64 * h + 32 + 16 * is + j]; // ql_b
        else
            val = blk[128 + 32 * h + 16 * is + j]; // qh
        qq[row * (U * 48) + plane * (U * 16) + (4 * kb + v) * 16 + j] = val;
    }
    if (t < 16) {
        int v = t >> 2, tt = t & 3;
        int h = v >> 1, is = v & 1;
        scq[b * 16 + t] = (int8_t)blk[192 + 8 * h + is + 2 * tt];
    }
    if (t == 0) {
        dq[2 * b] = blk[208];
        dq[2 * b + 1] = blk[209];
    }
}

// Q8_0: one thread per quant byte.  Block (row n, kb) is half kb&1 of unit
// kb/2 of row n of the padded [N][Kp] layout; byte i sits in plane
// (32*(kb&1) + i) / 16.  The destination is zeroed beforehand so the padding
// holds zero quants and zero scales.
extern "C" __global__ __launch_bounds__(256) void realm_repack_q80(
    const uint8_t *__restrict__ raw, uint8_t *__restrict__ dq, int8_t *__restrict__ qq,
    long long nblocks, int kb_per_row, int kp)
{
    long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long b = gid >> 5;
    if (b >= nblocks)
        return;
    int i = (int)(gid & 31);
    long long n = b / kb_per_row;
    int kb = (int)(b - n * kb_per_row);
    const uint8_t *blk = raw + b * Q80_BLOCK_BYTES;
    int ub = 32 * (kb & 1) + i; // byte of the 64-byte unit
    long long U = kp / 64;
    qq[n * kp + (ub >> 4) * (U * 16) + (kb >> 1) * 16 + (ub & 15)] = (int8_t)blk[2 + i];
    if (i < 2)
        dq[(n * (kp / 32) + kb) * 2 + i] = blk[i];
}

// The 32-element block formats of the reference (crates/realm-core/src/
// quant.rs:10-70, 226-370): Q4_0 (type 2, 18 B), Q4_1 (3, 20 B), Q5_0 (6,
// 22 B), Q5_1 (7, 24 B), Q8_1 (9, 36 B).  Element i of a block is q' s
// (+ delta for Q4_1, Q5_1, Q8_1) with s, delta the block's f16 fields and q'
// the small integer block32_q returns.
REALM_DEV int block32_bytes(int type)
{
    return type == 2 ? 18 : type == 3 ? 20 : type == 6 ? 22 : type == 7 ? 24 : 36;
}
REALM_DEV bool block32_delta(int type) { return type == 3 || type == 7 || type == 9; }
REALM_DEV int block32_q(int type, const uint8_t *b, int i)
{
    const bool delta = block32_delta(type);
    if (type == 2 || type == 3) {
        const uint8_t byte = b[(delta ? 4 : 2) + (i & 15)];
        return (i < 16 ? (byte & 0x0F) : (byte >> 4)) - 8;
    }
    if (type == 6 || type == 7) {
        const uint8_t *qh = b + (delta ? 4 : 2), *ql = qh + 4;
        const int lo = (i & 1) ? (ql[i >> 1] >> 4) : (ql[i >> 1] & 0x0F);
        const int sh = 4 * ((i & 3) >= 2) + (type == 6 ? 2 * ((i >> 2) & 1) : 0);
        return (lo | (((qh[i >> 3] >> sh) & 1) << 4)) - 16;
    }
    return (int8_t)b[4 + i];
}

// Bit-exact dequantization, one thread per output element.  Products and
// sums are separate f32 roundings (__fmul_rn / __fadd_rn), as the
// reference's mul-then-add.
extern "C" __global__ __launch_bounds__(256) void realm_dequant_q32(const uint8_t *raw, float *y,
                                                                   long long nb, int type)
{
    const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
    if (e >= nb * 32)
        return;
    const int i = (int)(e & 31);
    const uint8_t *b = raw + (e >> 5) * block32_bytes(type);
    const float s = realm::f16_bits_to_f32(b[0] | (b[1] << 8));
    const bool delta = block32_delta(type);
    const float d = delta ? realm::f16_bits_to_f32(b[2] | (b[3] << 8)) : 0.f;
    const float t = __fmul_rn((float)block32_q(type, b, i), s);
    y[e] = delta ? __fadd_rn(t, d) : t;
}

// Registration of a 32-element format as resident weights ("q8m"): q' as
// int8 in the Q8_0 layout (realm_repack_q80: row n, block kb, byte i in
// plane (32 (kb & 1) + i) / 16 of unit kb / 2), the f16 scale in the Q8_0
// scale stream and the f16 delta (zero for Q4_0 and Q5_0) in a stream of the
// same shape.  1.125 bytes per weight against 4 for f32; q' s + delta
// reproduces the reference's values exactly.  The destination is zeroed
// beforehand (padding: zero quants, scales and deltas).
extern "C" __global__ __launch_bounds__(256) void realm_repack_q32(
    const uint8_t *__restrict__ raw, uint8_t *__restrict__ dq, int8_t *__restrict__ qq,
    uint8_t *__restrict__ mq, long long nblocks, int kb_per_row, int kp, int type)
{
    const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long b = gid >> 5;
    if (b >= nblocks)
        return;
    const int i = (int)(gid & 31);
    const long long n = b / kb_per_row;
    const int kb = (int)(b - n * kb_per_row);
    const uint8_t *blk = raw + b * block32_bytes(type);
    const int ub = 32 * (kb & 1) + i;
    const long long U = kp / 64;
    qq[n * kp + (ub >> 4) * (U * 16) + (kb >> 1) * 16 + (ub & 15)] = (int8_t)block32_q(type, blk, i);
    const long long si = (n * (kp / 32) + kb) * 2;
    if (i < 2)
        dq[si + i] = blk[i];
    else if (i < 4 && block32_delta(type))
        mq[si + i - 2] = blk[i];
}

// A q8m matrix back to f32 W [n][k] for the dense products of larger
// batches: q' s (+ delta), the reference's roundings, so bit-exact with
// realm_dequant_q32 on the raw blocks.
extern "C" __global__ __launch_bounds__(256) void realm_dequant_q8m(
    const uint8_t *__restrict__ dq, const int8_t *__restrict__ qq, const uint8_t *__restrict__ mq,
    float *__restrict__ y, long long n, int k, int kp, int type)
{
    const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
    if (e >= n * k)
        return;
    const long long row = e / k;
    const int kk = (int)(e - row * k), qi = kk & 63;
    const long long U = kp / 64;
    const int q = qq[row * kp + (qi >> 4) * (U * 16) + (kk >> 6) * 16 + (qi & 15)];
    const long long si = (row * (kp / 32) + (kk >> 5)) * 2;
    const float s = realm::f16_bits_to_f32(dq[si] | (dq[si + 1] << 8));
    const float t = __fmul_rn((float)q, s);
    y[e] = block32_delta(type) ? __fadd_rn(t, realm::f16_bits_to_f32(mq[si] | (mq[si + 1] << 8)))
                               : t;
}

// The reference's own 256-element Q2_K (type 10, 116 B), Q3_K (11, 196 B),
// Q5_K (13, 178 B) and Q8_K (15, 292 B) blocks (crates/realm-core/src/
// quant.rs:71-95, 200-222, their #[repr(C)] sizes, not ggml's), dequantized
// as quant.rs:453-638 does, one thread per output element; separate f32
// roundings (__fmul_rn / __fadd_rn) in the reference's left-to-right order:
//   Q2_K: d * sc * q + dmin, q = 2 bits of qs[i/4] | bit of qh[i/8] << 2, - 2;
//         sc = nibble (i/16)%2 of scales[i/32]
//   Q3_K: the same bits, - 4; sc = (scales[i/32] >> 2((i/8)%4)) & 63
//   Q5_K: d * scales[i/16] * q for i < 128, q = int8(ql[i] | (qh nibble
//         (i%16)/4 %2 of qh[2(i/16) + (i%16)/8]) << 4); elements 128..255 are
//         never written by the reference (ql holds 128 bytes) and stay 0
//   Q8_K: d * sc * quants[i] + dmin, sc = nibble (i/8)%2 of scales[i/16]
extern "C" __global__ __launch_bounds__(256) void realm_dequant_kq(const uint8_t *raw, float *y,
                                                                  long long nb, int type)
{
    const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
    if (e >= nb * 256)
        return;
    const int i = (int)(e & 255);
    const int bb = type == 10 ? 116 : type == 11 ? 196 : type == 13 ? 178 : 292;
    const uint8_t *b = raw + (e >> 8) * bb;
    if (type == 13) {
        if (i >= 128) {
            y[e] = 0.f;
            return;
        }
        const int l = i >> 4, k = i & 15;
        const int qhv = (b[128 + 2 * l + (k >> 3)] >> (4 * ((k & 7) >> 2))) & 0xF;
        const int q = (int8_t)(uint8_t)(b[i] | ((qhv << 4) & 0xFF));
        const float d = realm::f16_bits_to_f32(b[176] | (b[177] << 8));
        y[e] = __fmul_rn(__fmul_rn(d, (float)(int8_t)b[160 + l]), (float)q);
        return;
    }
    const int off = type == 15 ? 288 : 0;
    const float d = realm::f16_bits_to_f32(b[off] | (b[off + 1] << 8));
    const float dmin = realm::f16_bits_to_f32(b[off + 2] | (b[off + 3] << 8));
    int sc, q;
    if (type == 15) {
        const int l = i >> 3, sbyte = b[256 + (l >> 1)];
        sc = (l & 1) ? (sbyte >> 4) : (sbyte & 0xF);
        q = (int8_t)b[i];
    } else {
        const uint8_t *scales = b + 4;
        const uint8_t *qh = scales + (type == 10 ? 16 : 32), *qs = qh + 32;
        const int qsb = (qs[i >> 2] >> ((i & 3) * 2)) & 3, qhb = (qh[i >> 3] >> (i & 7)) & 1;
        if (type == 10) {
            const int l = i >> 4, sbyte = scales[l >> 1];
            sc = (l & 1) ? (sbyte >> 4) : (sbyte & 0xF);
            q = (qsb | (qhb << 2)) - 2;
        } else {
            const int l = i >> 3;
            sc = (scales[l >> 2] >> ((l & 3) * 2)) & 0x3F;
            q = (qsb | (qhb << 2)) - 4;
        }
    }
    y[e] = __fadd_rn(__fmul_rn(__fmul_rn(d, (float)sc), (float)q), dmin);
}

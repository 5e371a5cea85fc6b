/*
 * realm_oracle.c -- CPU restatement of Realm's quantized compute path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP implementation, never
 * part of the product.  Built with -ffp-contract=off so that every `a*b - c`
 * is a separate multiply and subtract, as in the reference's Rust (which
 * never contracts to FMA).  Citations are to the reference checkout.
 */
#include "realm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- f16 */

/* IEEE binary16 -> binary32, exact (half 2.7.1 f16::to_f32, used by
 * crates/realm-core/src/quant.rs:134-135).  Subnormals are exact
 * (mantissa * 2^-24); NaN is returned quiet with its payload kept. */
float ro_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    float f;
    if (exp == 0) {
        f = ldexpf((float)man, -24);
        return (h & 0x8000u) ? -f : f;
    }
    if (exp == 31)
        bits = sign | 0x7F800000u | (man ? (0x400000u | (man << 13)) : 0u);
    else
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    memcpy(&f, &bits, 4);
    return f;
}

/* binary32 -> binary16 with round-to-nearest-even (half::f16::from_f32, used
 * by the reference tests to build blocks, e.g. quant.rs:978-979). */
uint16_t ro_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFF)
        return (uint16_t)(sign | 0x7C00u | (man ? (0x200u | (man >> 13)) : 0u));
    int e = (int)exp - 127 + 15;
    if (e >= 31)
        return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10)
            return (uint16_t)sign;
        man |= 0x800000u;
        int shift = 14 - e;
        uint32_t hm = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (hm & 1u)))
            hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t hm = man >> 13;
    uint32_t rem = man & 0x1FFFu;
    uint32_t out = sign | ((uint32_t)e << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u)))
        out++; /* a carry out of the mantissa correctly bumps the exponent */
    return (uint16_t)out;
}

/* ------------------------------------------------------------- dequant */

/* crates/realm-core/src/quant.rs:110-122 (get_scale_min_k4): 8 six-bit
 * (scale, min) pairs packed in 12 bytes. */
void ro_get_scale_min_k4(int j, const uint8_t *s, uint8_t *sc, uint8_t *m)
{
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* crates/realm-core/src/quant.rs:127-187 (dequantize_q4_k).  Four groups of
 * 64: byte qs[32g+j] holds element 64g+j in its low nibble (scale pair 2g)
 * and element 64g+32+j in its high nibble (pair 2g+1).
 * y = fl(fl(d*sc) * q) - fl(dmin*m), multiply then subtract. */
int ro_dequantize_q4_k(const ro_block_q4_k *b, float *y)
{
    float d = ro_f16_to_f32(b->d);
    float dmin = ro_f16_to_f32(b->dmin);
    for (int g = 0; g < 4; ++g) {
        uint8_t sc, m;
        ro_get_scale_min_k4(2 * g, b->scales, &sc, &m);
        float d1 = d * (float)sc;
        float m1 = dmin * (float)m;
        ro_get_scale_min_k4(2 * g + 1, b->scales, &sc, &m);
        float d2 = d * (float)sc;
        float m2 = dmin * (float)m;
        for (int j = 0; j < 32; ++j) {
            uint8_t q = b->qs[32 * g + j];
            y[64 * g + j] = d1 * (float)(q & 0xF) - m1;
        }
        for (int j = 0; j < 32; ++j) {
            uint8_t q = b->qs[32 * g + j];
            y[64 * g + 32 + j] = d2 * (float)(q >> 4) - m2;
        }
    }
    return RO_OK;
}

/* Six-bit Q6_K value t (0..3) of lane l in one 128-element half: low nibble
 * from ql[l] (t=0,2) or ql[l+32] (t=1,3), high 2 bits from qh[l] bits 2t. */
static int q6_value(const uint8_t *ql, const uint8_t *qh, int l, int t)
{
    uint8_t lo = (t & 1) ? ql[l + 32] : ql[l];
    lo = (t & 2) ? (uint8_t)(lo >> 4) : (uint8_t)(lo & 0xF);
    uint8_t hi = (uint8_t)((qh[l] >> (2 * t)) & 3);
    return (int)(int8_t)(uint8_t)(lo | (hi << 4)) - 32;
}

/* crates/realm-core/src/quant.rs:393-451 (dequantize_q6_k).  Half h covers
 * elements 128h..128h+127 with ql[64h..], qh[32h..], scales[8h..];
 * y[128h + l + 32t] = fl(fl(d*sc[8h + l/16 + 2t]) * q). */
int ro_dequantize_q6_k(const ro_block_q6_k *b, float *y)
{
    float d = ro_f16_to_f32(b->d);
    for (int h = 0; h < 2; ++h) {
        const uint8_t *ql = b->ql + 64 * h;
        const uint8_t *qh = b->qh + 32 * h;
        const int8_t *sc = b->scales + 8 * h;
        for (int l = 0; l < 32; ++l) {
            int is = l / 16;
            for (int t = 0; t < 4; ++t) {
                int q = q6_value(ql, qh, l, t);
                y[128 * h + l + 32 * t] = d * (float)sc[is + 2 * t] * (float)q;
            }
        }
    }
    return RO_OK;
}

/* crates/realm-core/src/quant.rs:371-387 (dequantize_q8_0): y = q * d. */
int ro_dequantize_q8_0(const ro_block_q8_0 *b, float *y)
{
    float s = ro_f16_to_f32(b->scale);
    for (int i = 0; i < 32; ++i)
        y[i] = (float)b->quants[i] * s;
    return RO_OK;
}

/* crates/realm-core/src/quant.rs:663-770 (dequantize_tensor) for the three
 * formats of this path.  Q4_K validates byte length (InvalidFormat) and
 * element count (InvalidShape).  Q6_K and Q8_0 validate nothing: a trailing
 * partial block is ignored, elements beyond the last block stay 0, and an
 * element_count smaller than the blocks' output makes the reference panic. */
/* The 32-element block formats, as the reference lays them out and
 * dequantizes them (crates/realm-core/src/quant.rs:10-70, 226-370):
 *   Q4_0 (18 B): f16 scale, 16 B nibbles; y[i] = (lo(b[i]) - 8) s,
 *                y[i + 16] = (hi(b[i]) - 8) s
 *   Q4_1 (20 B): f16 scale, f16 delta, nibbles as Q4_0, then + delta
 *   Q5_0 (22 B): f16 scale, qh[4], ql[16]; element i: nibble i%2 of ql[i/2],
 *                high bit (qh[i/8] >> (4 ((i%4) >= 2) + 2 ((i/4)%2))) & 1,
 *                y = (q - 16) s
 *   Q5_1 (24 B): f16 scale, f16 delta, qh[4], ql[16]; high bit
 *                (qh[i/8] >> 4 ((i%4) >= 2)) & 1, y = (q - 16) s + delta
 *   Q8_1 (36 B): f16 scale, f16 delta, 32 int8; y = q s + delta
 * Each product and sum rounds to f32 on its own (no fused multiply-add). */
int ro_block32_bytes(int type)
{
    switch (type) {
    case RO_GGML_Q4_0: return 18;
    case RO_GGML_Q4_1: return 20;
    case RO_GGML_Q5_0: return 22;
    case RO_GGML_Q5_1: return 24;
    case RO_GGML_Q8_1: return 36;
    default: return 0;
    }
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* The reference's own 256-element Q2_K, Q3_K, Q5_K and Q8_K blocks
 * (crates/realm-core/src/quant.rs:71-95, 200-222; #[repr(C)] sizes, not
 * ggml's), dequantized as quant.rs:453-638 does:
 *   Q2_K (116 B: d, dmin, scales[16], qh[32], qs[64]): element i of group
 *        l = i/16 has q = ((qs[i/4] >> 2(i%4)) & 3 | ((qh[i/8] >> (i%8)) & 1)
 *        << 2) - 2 and scale nibble l%2 of scales[l/2]; y = d sc q + dmin
 *   Q3_K (196 B: d, dmin, scales[32], qh[32], qs[128]): group l = i/8, scale
 *        (scales[l/4] >> 2(l%4)) & 63, q = (2 qs bits | qh bit << 2) - 4 with
 *        the Q2_K indexing; y = d sc q + dmin
 *   Q5_K (178 B: ql[128], qh[32], scales[16] i8, d): only elements 0..127
 *        are written (ql has 128 bytes; the reference's loop stops there and
 *        leaves the rest of its zeroed output); element i = 16 l + k has
 *        q = int8(ql[i] | ((qh[2l + k/8] >> 4((k%8)/4)) & 15) << 4),
 *        y = d scales[l] q
 *   Q8_K (292 B: quants[256] i8, scales[32], d, dmin): group l = i/8,
 *        scale nibble l%2 of scales[l/2]; y = d sc q + dmin
 * Each product and sum rounds to f32 on its own, left to right. */
int ro_kquant_bytes(int type)
{
    switch (type) {
    case RO_GGML_Q2_K: return 116;
    case RO_GGML_Q3_K: return 196;
    case RO_GGML_Q5_K: return 178;
    case RO_GGML_Q8_K: return 292;
    default: return 0;
    }
}

static void dequantize_kquant(int type, const uint8_t *b, float *y)
{
    volatile float t; /* keeps each rounding step separate */
    if (type == RO_GGML_Q5_K) {
        const uint8_t *ql = b, *qh = b + 128;
        const int8_t *scales = (const int8_t *)(b + 160);
        const float d = ro_f16_to_f32(rd16(b + 176));
        for (int i = 0; i < 256; ++i)
            y[i] = 0.0f;
        for (int l = 0; l < 8; ++l) /* l >= 8: ql index past 127, loop stops */
            for (int k = 0; k < 16; ++k) {
                const int i = 16 * l + k;
                const int qhv = (qh[2 * l + k / 8] >> (4 * ((k % 8) / 4))) & 0xF;
                const int8_t q = (int8_t)(uint8_t)(ql[i] | ((qhv << 4) & 0xFF));
                t = d * (float)scales[l];
                y[i] = t * (float)q;
            }
        return;
    }
    const int off = type == RO_GGML_Q8_K ? 288 : 0; /* d, dmin */
    const float d = ro_f16_to_f32(rd16(b + off)), dmin = ro_f16_to_f32(rd16(b + off + 2));
    for (int i = 0; i < 256; ++i) {
        int sc, q;
        if (type == RO_GGML_Q8_K) {
            const int l = i / 8, sb = b[256 + l / 2];
            sc = (l % 2 == 0) ? (sb & 0xF) : (sb >> 4);
            q = (int8_t)b[i];
        } else {
            const uint8_t *scales = b + 4;
            const uint8_t *qh = scales + (type == RO_GGML_Q2_K ? 16 : 32), *qs = qh + 32;
            const int qsb = (qs[i / 4] >> ((i % 4) * 2)) & 3, qhb = (qh[i / 8] >> (i % 8)) & 1;
            if (type == RO_GGML_Q2_K) {
                const int l = i / 16, sb = scales[l / 2];
                sc = (l % 2 == 0) ? (sb & 0xF) : (sb >> 4);
                q = (qsb | (qhb << 2)) - 2;
            } else {
                const int l = i / 8;
                sc = (scales[l / 4] >> ((l % 4) * 2)) & 0x3F;
                q = (qsb | (qhb << 2)) - 4;
            }
        }
        t = d * (float)sc;
        t = t * (float)q;
        y[i] = (float)(t + dmin);
    }
}

static void dequantize_block32(int type, const uint8_t *b, float *y)
{
    volatile float t; /* keeps each rounding step separate */
    const float s = ro_f16_to_f32(rd16(b));
    if (type == RO_GGML_Q4_0 || type == RO_GGML_Q4_1) {
        const int q1 = type == RO_GGML_Q4_1;
        const float d = q1 ? ro_f16_to_f32(rd16(b + 2)) : 0.0f;
        const uint8_t *qs = b + (q1 ? 4 : 2);
        for (int i = 0; i < 16; ++i) {
            t = (float)((int)(qs[i] & 0x0F) - 8) * s;
            y[i] = q1 ? (float)(t + d) : t;
            t = (float)((int)(qs[i] >> 4) - 8) * s;
            y[i + 16] = q1 ? (float)(t + d) : t;
        }
    } else if (type == RO_GGML_Q5_0 || type == RO_GGML_Q5_1) {
        const int q1 = type == RO_GGML_Q5_1;
        const float d = q1 ? ro_f16_to_f32(rd16(b + 2)) : 0.0f;
        const uint8_t *qh = b + (q1 ? 4 : 2), *ql = qh + 4;
        for (int i = 0; i < 32; ++i) {
            const int lo = (i % 2 == 0) ? (ql[i / 2] & 0x0F) : (ql[i / 2] >> 4);
            const int sh = 4 * ((i % 4) >= 2) + (q1 ? 0 : 2 * ((i / 4) % 2));
            const int hi = (qh[i / 8] >> sh) & 1;
            t = (float)((lo | (hi << 4)) - 16) * s;
            y[i] = q1 ? (float)(t + d) : t;
        }
    } else { /* Q8_1 */
        const float d = ro_f16_to_f32(rd16(b + 2));
        for (int i = 0; i < 32; ++i) {
            t = (float)(int8_t)b[4 + i] * s;
            y[i] = (float)(t + d);
        }
    }
}

int ro_dequantize_tensor(const uint8_t *data, size_t nbytes, int type,
                         size_t element_count, float *out)
{
    memset(out, 0, element_count * sizeof(float));
    if (type == RO_GGML_Q4_K) {
        if (nbytes % sizeof(ro_block_q4_k))
            return RO_MODEL_PARSE_ERROR;
        size_t nb = nbytes / sizeof(ro_block_q4_k);
        if (element_count != nb * RO_QK_K)
            return RO_INVALID_ARGUMENT;
        for (size_t i = 0; i < nb; ++i) {
            ro_block_q4_k b;
            memcpy(&b, data + i * sizeof b, sizeof b);
            ro_dequantize_q4_k(&b, out + i * RO_QK_K);
        }
        return RO_OK;
    }
    if (type == RO_GGML_Q6_K) {
        size_t nb = nbytes / sizeof(ro_block_q6_k);
        if (nb * RO_QK_K > element_count)
            return RO_PANIC;
        for (size_t i = 0; i < nb; ++i) {
            ro_block_q6_k b;
            memcpy(&b, data + i * sizeof b, sizeof b);
            ro_dequantize_q6_k(&b, out + i * RO_QK_K);
        }
        return RO_OK;
    }
    if (type == RO_GGML_Q8_0) {
        size_t nb = nbytes / sizeof(ro_block_q8_0);
        if (nb * RO_QK8_0 > element_count)
            return RO_PANIC;
        for (size_t i = 0; i < nb; ++i) {
            ro_block_q8_0 b;
            memcpy(&b, data + i * sizeof b, sizeof b);
            ro_dequantize_q8_0(&b, out + i * RO_QK8_0);
        }
        return RO_OK;
    }
    if (ro_kquant_bytes(type)) { /* quant.rs:722-756, 859-892: no size validation */
        const size_t bb = (size_t)ro_kquant_bytes(type), nb = nbytes / bb;
        if (nb * 256 > element_count)
            return RO_PANIC;
        for (size_t i = 0; i < nb; ++i)
            dequantize_kquant(type, data + i * bb, out + i * 256);
        return RO_OK;
    }
    if (ro_block32_bytes(type)) { /* quant.rs:773-856: no size validation */
        const size_t bb = (size_t)ro_block32_bytes(type), nb = nbytes / bb;
        if (nb * 32 > element_count)
            return RO_PANIC;
        for (size_t i = 0; i < nb; ++i)
            dequantize_block32(type, data + i * bb, out + i * 32);
        return RO_OK;
    }
    return RO_GENERIC_FAILURE; /* format not restated here */
}

/* --------------------------------------------------------------- fused */

/* NaN/Inf super-block scales are replaced by constants in fused.rs
 * (crates/realm-compute-cpu/src/fused.rs:276-285, 1171-1175). */
static float fix_scale(float v, float fallback, int enable)
{
    return (enable && !isfinite(v)) ? fallback : v;
}

/* crates/realm-compute-cpu/src/fused.rs:229-374 (fused_dequant_matmul_q4k),
 * accumulation order of the portable path q4k_accumulate_scalar
 * (fused.rs:156-196): per byte j of a group, low nibble then high nibble. */
int ro_fused_q4k(const ro_block_q4_k *blocks, size_t nblocks, const float *input,
                 size_t input_len, float *out, size_t batch, size_t n, size_t k,
                 int nan_fallback)
{
    if (k % RO_QK_K)
        return RO_INVALID_ARGUMENT;
    size_t nbr = k / RO_QK_K;
    if (nblocks != n * nbr)
        return RO_INVALID_ARGUMENT;
    if (input_len < batch * k)
        return RO_PANIC;
    for (size_t bi = 0; bi < batch; ++bi) {
        const float *x = input + bi * k;
        for (size_t o = 0; o < n; ++o) {
            float acc = 0.0f;
            for (size_t kb = 0; kb < nbr; ++kb) {
                const ro_block_q4_k *b = &blocks[o * nbr + kb];
                float d = fix_scale(ro_f16_to_f32(b->d), 0.00000006f, nan_fallback);
                float dmin = fix_scale(ro_f16_to_f32(b->dmin), 0.00000024f, nan_fallback);
                for (int g = 0; g < 4; ++g) {
                    uint8_t sc, m;
                    ro_get_scale_min_k4(2 * g, b->scales, &sc, &m);
                    float d1 = d * (float)sc, m1 = dmin * (float)m;
                    ro_get_scale_min_k4(2 * g + 1, b->scales, &sc, &m);
                    float d2 = d * (float)sc, m2 = dmin * (float)m;
                    const float *xg = x + kb * RO_QK_K + 64 * g;
                    for (int j = 0; j < 32; ++j) {
                        uint8_t q = b->qs[32 * g + j];
                        acc += (d1 * (float)(q & 0xF) - m1) * xg[j];
                        acc += (d2 * (float)(q >> 4) - m2) * xg[32 + j];
                    }
                }
            }
            out[bi * n + o] = acc;
        }
    }
    return RO_OK;
}

/* crates/realm-compute-cpu/src/fused.rs:1128-1259 (fused_dequant_matmul_q6k)
 * with the portable 4-value step q6k_process_4_values (fused.rs:949-970):
 * four products, summed left to right, added to the accumulator. */
int ro_fused_q6k(const ro_block_q6_k *blocks, size_t nblocks, const float *input,
                 size_t input_len, float *out, size_t batch, size_t n, size_t k,
                 int nan_fallback)
{
    if (k % RO_QK_K)
        return RO_INVALID_ARGUMENT;
    size_t nbr = k / RO_QK_K;
    if (nblocks != n * nbr)
        return RO_INVALID_ARGUMENT;
    if (input_len < batch * k)
        return RO_PANIC;
    for (size_t bi = 0; bi < batch; ++bi) {
        const float *x = input + bi * k;
        for (size_t o = 0; o < n; ++o) {
            float acc = 0.0f;
            for (size_t kb = 0; kb < nbr; ++kb) {
                const ro_block_q6_k *b = &blocks[o * nbr + kb];
                float d = fix_scale(ro_f16_to_f32(b->d), 0.00000006f, nan_fallback);
                for (int h = 0; h < 2; ++h) {
                    const uint8_t *ql = b->ql + 64 * h;
                    const uint8_t *qh = b->qh + 32 * h;
                    const int8_t *sc = b->scales + 8 * h;
                    const float *xh = x + kb * RO_QK_K + 128 * h;
                    for (int l = 0; l < 32; ++l) {
                        int is = l / 16;
                        float p[4];
                        for (int t = 0; t < 4; ++t) {
                            int q = q6_value(ql, qh, l, t);
                            p[t] = d * (float)sc[is + 2 * t] * (float)q * xh[l + 32 * t];
                        }
                        acc += p[0] + p[1] + p[2] + p[3];
                    }
                }
            }
            out[bi * n + o] = acc;
        }
    }
    return RO_OK;
}

/* crates/realm-compute-cpu/src/fused.rs:2451-2554 (fused_dequant_matmul_q80):
 * ceil(n*k/32) blocks expected, input length checked, K tails handled with a
 * per-row stride of ceil(k/32) blocks (block indices past the end skipped). */
int ro_fused_q80(const ro_block_q8_0 *blocks, size_t nblocks, const float *input,
                 size_t input_len, float *out, size_t batch, size_t n, size_t k)
{
    size_t expected = (n * k + RO_QK8_0 - 1) / RO_QK8_0;
    if (nblocks != expected)
        return RO_INVALID_ARGUMENT;
    if (input_len != batch * k)
        return RO_INVALID_ARGUMENT;
    size_t nkb = (k + RO_QK8_0 - 1) / RO_QK8_0;
    for (size_t o = 0; o < n; ++o) {
        for (size_t bi = 0; bi < batch; ++bi) {
            float sum = 0.0f;
            for (size_t kb = 0; kb < nkb; ++kb) {
                size_t k0 = kb * RO_QK8_0;
                size_t k1 = k0 + RO_QK8_0 < k ? k0 + RO_QK8_0 : k;
                size_t bidx = o * nkb + kb;
                if (bidx >= nblocks)
                    continue;
                float s = ro_f16_to_f32(blocks[bidx].scale);
                for (size_t i = 0; i < k1 - k0; ++i)
                    sum += ((float)blocks[bidx].quants[i] * s) * input[bi * k + k0 + i];
            }
            out[bi * n + o] = sum;
        }
    }
    return RO_OK;
}

/* --------------------------------------------------------------- dense */

/* crates/realm-compute-cpu/src/gemm.rs:83-143 (matmul_transposed):
 * c[i,j] = sum_l a[i,l]*bt[j,l], one f32 accumulator, l ascending. */
int ro_matmul_transposed(const float *a, size_t a_len, const float *bt,
                         size_t bt_len, float *c, size_t m, size_t k, size_t n)
{
    if (a_len != m * k || bt_len != n * k)
        return RO_INVALID_ARGUMENT;
    for (size_t i = 0; i < m; ++i)
        for (size_t j = 0; j < n; ++j) {
            float s = 0.0f;
            for (size_t l = 0; l < k; ++l)
                s += a[i * k + l] * bt[j * k + l];
            c[i * n + j] = s;
        }
    return RO_OK;
}

/* crates/realm-compute-cpu/src/gemm.rs:11-74 (matmul_f32): C = A*B with
 * A [m,k], B [k,n]; per element the products are added in l order. */
int ro_matmul_f32(const float *a, size_t a_len, const float *b, size_t b_len,
                  float *c, size_t m, size_t k, size_t n)
{
    if (a_len != m * k || b_len != k * n)
        return RO_INVALID_ARGUMENT;
    for (size_t i = 0; i < m; ++i)
        for (size_t j = 0; j < n; ++j) {
            float s = 0.0f;
            for (size_t l = 0; l < k; ++l)
                s += a[i * k + l] * b[l * n + j];
            c[i * n + j] = s;
        }
    return RO_OK;
}

/* crates/realm-compute-cpu/src/candle_cpu_backend.rs:92-114 (q4k), :137-156
 * (q6k), :305-324 (q80): dequantize every block with quant.rs, then
 * matmul_transposed(input [batch,k], W [n,k]).  Shape errors come only from
 * the matmul (input length, n*k == dequantized length).  The Candle GEMM's
 * own summation order is replaced by gemm.rs's sequential order. */
int ro_candle_fused(int type, const void *blocks, size_t nblocks,
                    const float *input, size_t input_len, float *out,
                    size_t batch, size_t n, size_t k)
{
    size_t per = (type == RO_GGML_Q8_0 || ro_block32_bytes(type)) ? RO_QK8_0 : RO_QK_K;
    size_t total = nblocks * per;
    float *w = (float *)malloc((total ? total : 1) * sizeof(float));
    if (!w)
        return RO_GENERIC_FAILURE;
    for (size_t i = 0; i < nblocks; ++i) {
        if (type == RO_GGML_Q4_K)
            ro_dequantize_q4_k((const ro_block_q4_k *)blocks + i, w + i * per);
        else if (type == RO_GGML_Q6_K)
            ro_dequantize_q6_k((const ro_block_q6_k *)blocks + i, w + i * per);
        else if (type == RO_GGML_Q8_0)
            ro_dequantize_q8_0((const ro_block_q8_0 *)blocks + i, w + i * per);
        else if (ro_kquant_bytes(type))
            dequantize_kquant(type, (const uint8_t *)blocks + i * ro_kquant_bytes(type),
                              w + i * per);
        else if (ro_block32_bytes(type))
            dequantize_block32(type, (const uint8_t *)blocks + i * ro_block32_bytes(type),
                               w + i * per);
        else {
            free(w);
            return RO_GENERIC_FAILURE;
        }
    }
    int rc = ro_matmul_transposed(input, input_len, w, total, out, batch, k, n);
    free(w);
    return rc;
}

/* ---------------------------------------------------------------- LoRA */

/* crates/realm-runtime/src/lora.rs:91-144 (LoRAManager::apply_to_weights)
 * with scale() = alpha / rank (lora.rs:49-52):
 *   delta[i,j] = fl(sum_k B[i*r+k]*A[k*in+j]) * scale  (index-guarded)
 *   out = base; out[i] += delta[i] for i < min(len(base), out*in). */
int ro_lora_apply_to_weights(const float *base, size_t base_len, const float *A,
                             size_t a_len, const float *B, size_t b_len,
                             size_t rank, float alpha, size_t out_dim, size_t in_dim,
                             float *out)
{
    float scale = alpha / (float)rank;
    memcpy(out, base, base_len * sizeof(float));
    size_t lim = base_len < out_dim * in_dim ? base_len : out_dim * in_dim;
    for (size_t i = 0; i < out_dim; ++i)
        for (size_t j = 0; j < in_dim; ++j) {
            float s = 0.0f;
            for (size_t r = 0; r < rank; ++r) {
                size_t ai = r * in_dim + j, bi = i * rank + r;
                if (ai < a_len && bi < b_len)
                    s += B[bi] * A[ai];
            }
            size_t idx = i * in_dim + j;
            if (idx < lim)
                out[idx] += s * scale;
        }
    return RO_OK;
}

/* Unmerged form of the same delta, per token (the merged and unmerged forms
 * are equal by associativity; tests check that on small shapes). */
int ro_multi_lora_delta(const float *x, size_t batch, size_t k, size_t n,
                        const int32_t *ids, size_t n_adapters,
                        const float *const *a_ptrs, const float *const *b_ptrs,
                        const int32_t *ranks, const float *alphas, float *y)
{
    float *u = (float *)malloc(64 * 1024 * sizeof(float));
    if (!u)
        return RO_GENERIC_FAILURE;
    for (size_t t = 0; t < batch; ++t) {
        int32_t a = ids[t];
        if (a < 0 || (size_t)a >= n_adapters)
            continue;
        size_t r = (size_t)ranks[a];
        if (r > 64 * 1024) {
            free(u);
            return RO_INVALID_ARGUMENT;
        }
        const float *A = a_ptrs[a], *B = b_ptrs[a];
        float scale = alphas[a] / (float)r;
        for (size_t j = 0; j < r; ++j) {
            float s = 0.0f;
            for (size_t l = 0; l < k; ++l)
                s += A[j * k + l] * x[t * k + l];
            u[j] = s;
        }
        for (size_t o = 0; o < n; ++o) {
            float s = 0.0f;
            for (size_t j = 0; j < r; ++j)
                s += B[o * r + j] * u[j];
            y[t * n + o] += scale * s;
        }
    }
    free(u);
    return RO_OK;
}

/* ------------------------------------------------------------ checkers */

void ro_matvec_f64(const float *w, const float *x, double *y, size_t batch,
                   size_t n, size_t k)
{
    for (size_t b = 0; b < batch; ++b)
        for (size_t o = 0; o < n; ++o) {
            double s = 0.0;
            for (size_t l = 0; l < k; ++l)
                s += (double)w[o * k + l] * (double)x[b * k + l];
            y[b * n + o] = s;
        }
}

int ro_fused_parallel(int type, const void *blocks, const float *input, float *out,
                      size_t batch, size_t n, size_t k, int threads)
{
    size_t per = type == RO_GGML_Q8_0 ? RO_QK8_0 : RO_QK_K;
    size_t bpr = k / per;
    int used = 1;
#ifdef _OPENMP
    if (threads > 0)
        omp_set_num_threads(threads);
#pragma omp parallel
    {
#pragma omp single
        used = omp_get_num_threads();
        float *w = (float *)malloc(k * sizeof(float));
#pragma omp for schedule(static)
        for (long o = 0; o < (long)n; ++o) {
            for (size_t i = 0; i < bpr; ++i) {
                size_t bidx = (size_t)o * bpr + i;
                if (type == RO_GGML_Q4_K)
                    ro_dequantize_q4_k((const ro_block_q4_k *)blocks + bidx, w + i * per);
                else if (type == RO_GGML_Q6_K)
                    ro_dequantize_q6_k((const ro_block_q6_k *)blocks + bidx, w + i * per);
                else
                    ro_dequantize_q8_0((const ro_block_q8_0 *)blocks + bidx, w + i * per);
            }
            for (size_t b = 0; b < batch; ++b) {
                float s = 0.0f;
                for (size_t l = 0; l < k; ++l)
                    s += w[l] * input[b * k + l];
                out[b * n + o] = s;
            }
        }
        free(w);
    }
#else
    (void)threads;
    float *w = (float *)malloc(k * sizeof(float));
    for (size_t o = 0; o < n; ++o) {
        for (size_t i = 0; i < bpr; ++i) {
            size_t bidx = o * bpr + i;
            if (type == RO_GGML_Q4_K)
                ro_dequantize_q4_k((const ro_block_q4_k *)blocks + bidx, w + i * per);
            else if (type == RO_GGML_Q6_K)
                ro_dequantize_q6_k((const ro_block_q6_k *)blocks + bidx, w + i * per);
            else
                ro_dequantize_q8_0((const ro_block_q8_0 *)blocks + bidx, w + i * per);
        }
        for (size_t b = 0; b < batch; ++b) {
            float s = 0.0f;
            for (size_t l = 0; l < k; ++l)
                s += w[l] * input[b * k + l];
            out[b * n + o] = s;
        }
    }
    free(w);
#endif
    return used;
}

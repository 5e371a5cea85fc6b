// The exact f32 path for tokens whose activations the fast paths cannot
// represent: a non-finite element (NaN, +Inf, -Inf), or a range the integer /
// f16 activation scaling does not cover (a block max below 2^-60 or above
// 2^100, where a scale or its reciprocal would leave the normal range).
//
// For such a token the reference computes y[n] = sum_k W[n,k] x[k] in f32
// over the dequantized weights (crates/realm-compute-cpu/src/
// candle_cpu_backend.rs:92-114, 137-156, 305-324; fused.rs:229-374): a NaN
// in x gives NaN, an Inf gives +-Inf by the sign of the weights it meets, or
// NaN where it meets a zero weight or both signs.  The kernels flag the
// token while staging its activations and then recompute its rows here,
// element by element, with every weight dequantized exactly as quant.rs
// does (crates/realm-core/src/quant.rs:127-187, 371-387, 393-451; same
// operation order, no fused multiply-add), so the zero / sign / NaN pattern
// of the products is the reference's.  The result class of a sum of
// non-finite terms does not depend on the summation order; for the
// out-of-range finite tokens the sum is an ordinary f32 sum.
//
// This path is for rare inputs: it reads the weights element by element
// from the device layout of common.h.
#pragma once

#include "common.h"

namespace realm {

// Activation range the fast paths take per 32-element block (by its max
// |x|, zero blocks included); anything else goes through the exact path.
constexpr float EXACT_LO = 0x1p-60f;
constexpr float EXACT_HI = 0x1p100f;

REALM_DEV bool exact_needed(float amax, bool nonfinite)
{
    return nonfinite || (amax != 0.f && (amax < EXACT_LO || amax > EXACT_HI));
}

// Weight W[row][k] of a resident matrix (device layout of common.h), as the
// reference's dequantizer produces it.  K is the row length (KX: padded, Q8_0).
template <int FMT>
REALM_DEV float dev_weight(const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1,
                          const uint8_t *__restrict__ w2, int row, int k, int KX, int nan_fb)
{
#pragma clang fp contract(off)
    const int U = KX >> 6, u = k >> 6;
    if constexpr (FMT == 0) { // Q4_K
        const int B = KX >> 8;
        const uint32_t *h = reinterpret_cast<const uint32_t *>(w0 + ((size_t)row * B + (k >> 8)) * 16);
        const uint32_t h0 = h[0];
        const float d = fix_scale(f16_bits_to_f32(h0), 0.00000006f, nan_fb);
        const float dmin = fix_scale(f16_bits_to_f32(h0 >> 16), 0.00000024f, nan_fb);
        const uint32_t pr = q4k_dev_pair(h[1], h[2], h[3], u & 3);
        const int j = k & 63;
        const bool hi = j >= 32;
        const uint32_t sc = hi ? (pr >> 12) & 63u : pr & 63u;
        const uint32_t m = hi ? (pr >> 18) & 63u : (pr >> 6) & 63u;
        const int jb = j & 31;
        const uint32_t byte = w1[(size_t)row * U * 32 + (jb >> 4) * U * 16 + u * 16 + (jb & 15)];
        const uint32_t q = hi ? ((byte >> 4) ^ 8u) : (byte & 15u);
        const float d1 = d * (float)sc;
        const float m1 = dmin * (float)m;
        return d1 * (float)q - m1;
    } else if constexpr (FMT == 1) { // Q6_K
        const int B = KX >> 8;
        const int b = k >> 8, r = k & 255, hh = r >> 7, t = (r >> 5) & 3, l = r & 31;
        const int is = l >> 4, jj = l & 15, v = 2 * hh + is;
        const float d = fix_scale(
            f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(w0 + ((size_t)row * B + b) * 2)),
            0.00000006f, nan_fb);
        const int8_t sc = (int8_t)w1[((size_t)row * B + b) * 16 + v * 4 + t];
        const size_t q0 = (size_t)row * U * 48 + (size_t)(4 * b + v) * 16 + jj;
        const uint32_t qa = w2[q0 + (t & 1) * U * 16]; // ql plane 0 (t = 0, 2) or 1 (t = 1, 3)
        const uint32_t qh = w2[q0 + 2 * U * 16];
        const uint32_t lo = t < 2 ? (qa & 15u) : (qa >> 4);
        const int q = (int)(lo | (((qh >> (2 * t)) & 3u) << 4)) - 32;
        return d * (float)sc * (float)q;
    } else { // Q8_0; 3: the 32-element formats as int8 q, f16 scale, f16 delta (q8m)
        const size_t bi = (size_t)row * (KX >> 5) + (k >> 5);
        const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(w0 + bi * 2));
        const int qi = k & 63;
        const int8_t q = (int8_t)w1[(size_t)row * U * 64 + (qi >> 4) * U * 16 + u * 16 + (qi & 15)];
        if constexpr (FMT == 3)
            return (float)q * d + f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(w2 + bi * 2));
        return (float)q * d;
    }
}

// Activation k of one token row, f32 or bf16.
REALM_DEV float exact_x(const void *x, int bf16, size_t i)
{
    if (bf16)
        return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t *>(x)[i] << 16);
    return reinterpret_cast<const float *>(x)[i];
}

// Partial sum over k = k0, k0 + step, ... < K of W[row][k] x[k] (f32
// products and sums, no contraction); x is one token's row.
template <int FMT>
REALM_DEV float exact_dot(const void *w0, const void *w1, const void *w2, int row, int K, int KX,
                          const void *x, int bf16, int nan_fb, int k0, int step)
{
#pragma clang fp contract(off)
    float acc = 0.f;
    for (int k = k0; k < K; k += step)
        acc += dev_weight<FMT>((const uint8_t *)w0, (const uint8_t *)w1, (const uint8_t *)w2, row,
                               k, KX, nan_fb) *
               exact_x(x, bf16, (size_t)k);
    return acc;
}

// The same sum with eight products formed at a time (their loads in flight
// together), then added in k order: for kernels with registers to spare
// (the GEMVs' budget of 128 VGPRs would spill).
template <int FMT>
REALM_DEV float exact_dot_ilp(const void *w0, const void *w1, const void *w2, int row, int K,
                              int KX, const void *x, int bf16, int nan_fb, int k0, int step)
{
#pragma clang fp contract(off)
    constexpr int U = 8;
    float acc = 0.f;
    int k = k0;
    for (; k + (U - 1) * step < K; k += U * step) {
        float p[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            p[u] = dev_weight<FMT>((const uint8_t *)w0, (const uint8_t *)w1, (const uint8_t *)w2,
                                   row, k + u * step, KX, nan_fb) *
                   exact_x(x, bf16, (size_t)(k + u * step));
#pragma unroll
        for (int u = 0; u < U; ++u)
            acc += p[u];
    }
    for (; k < K; k += step)
        acc += dev_weight<FMT>((const uint8_t *)w0, (const uint8_t *)w1, (const uint8_t *)w2, row,
                               k, KX, nan_fb) *
               exact_x(x, bf16, (size_t)k);
    return acc;
}

// exact_dot of one (row, token) by the 64 lanes of a wave: lane l sums
// k = l, l + 64, ... in k order, then a butterfly adds the partial sums
// (IEEE addition commutes, so every lane ends with the same bits).
template <int FMT>
REALM_DEV float exact_dot_wave(const void *w0, const void *w1, const void *w2, int row, int K,
                               int KX, const void *x, int bf16, int nan_fb, int lane)
{
#pragma clang fp contract(off)
    float s = exact_dot_ilp<FMT>(w0, w1, w2, row, K, KX, x, bf16, nan_fb, lane, 64);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        s += __shfl_xor(s, off, 64);
    return s;
}

} // namespace realm

// Decode GEMV, 1-4 tokens: y[t][n] = sum_k W[n,k] x[t][k] for resident Q4_K /
// Q6_K / Q8_0 weights in the device layout of common.h, up to 4 matrices that
// share x per launch (rows concatenated: e.g. Q/K/V, or gate/up).
//
// Arithmetic: integer dot products.  Each workgroup first quantizes x per
// 32-element block b into two int8 planes, scale s_b = amax_b / 127:
//   xh = round(x / s_b),  xl = round((x - s_b*xh) * 254 / s_b)
//   x ~= s_b * (xh + xl/254),  |error| <= amax_b / (127*508) = 1.55e-5 * amax_b.
// Weights stay exact small integers (Q4_K 0..15, Q6_K 0..63 before the -32
// offset, Q8_0 -127..127), so v_dot4_i32_i8 accumulates 4 exact products per
// instruction in int32.  Per 32 (Q6_K: 16) weights the two int32 sums become
// s_b*(Ph + Pl/254) in f32 and take the block scales; the Q4_K min term and
// the Q6_K -32 offset use the exact integer sums of the quantized x.
//
// Work decomposition: a row is cut into U "units" of 64 weights (Q4_K: one
// 32-byte qs group + the block header; Q6_K: one 48-byte ql/qh group + 4
// sub-scales + d; Q8_0: two 34-byte blocks).  LPR lanes share a row; lane l
// owns units l, l+LPR, ... (UPL of them) of every row it visits, and a wave
// covers 64/LPR rows per pass.  The grid has at most one workgroup per CU;
// each wave strides over passes and keeps a ring of D passes in flight, all
// issued before its first pass is computed (the host picks D so that a
// wave's passes usually all fit: the whole weight stream is requested up
// front).  Quantized x lives in LDS as one 16-byte record per (unit, dword
// position), laid out [position][unit], so lanes of a wave read consecutive
// records (no bank conflicts).
#include "common.h"
#include "exact.h"
#include "kernel_args.h"

using namespace realm;
using realm::GemvArgs;

#define FMT_Q4K 0
#define FMT_Q6K 1
#define FMT_Q80 2
#define FMT_Q8M 3 // Q4_0, Q4_1, Q5_0, Q5_1, Q8_1: int8 q, f16 scale and delta per 32
// one metadata float4 per unit (two 32-element x blocks)
#define ONE_META(FMT) ((FMT) == FMT_Q80 || (FMT) == FMT_Q8M)

namespace {

REALM_DEV uint32_t word(const uint4 &v, int i)
{
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

REALM_DEV int dot4(uint32_t a, uint32_t b, int c)
{
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

template <int CTRL, int ROW_MASK>
REALM_DEV float dpp_f(float x)
{
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROW_MASK, 0xF,
                                           false));
}

// Sum over the LPR lanes of a lane group with DPP (quad swaps, row
// rotations, row broadcasts); the total lands in the group's last lane.
template <int LPR>
REALM_DEV float group_total(float v)
{
    v += dpp_f<0xB1, 0xF>(v);  // quad_perm [1,0,3,2]
    v += dpp_f<0x4E, 0xF>(v);  // quad_perm [2,3,0,1]
    v += dpp_f<0x124, 0xF>(v); // row_ror:4
    v += dpp_f<0x128, 0xF>(v); // row_ror:8  -> every lane holds its row's sum
    if (LPR >= 32)
        v += dpp_f<0x142, 0xA>(v); // row_bcast:15 into rows 1 and 3
    if (LPR >= 64)
        v += dpp_f<0x143, 0xC>(v); // row_bcast:31 into rows 2 and 3
    return v;
}


// Quantize x into LDS.  rec[pos * U + u] (int4) holds, for unit u and dword
// position pos, the xh and xl dwords its dot products need:
//   Q4_K / Q8_0 (unit = x blocks 2u, 2u+1; pos = i in 0..7):
//     (xh, xl of block 2u elements 4i..4i+3, xh, xl of block 2u+1 elements 4i..)
//   Q6_K (unit = 16-runs t = 0..3 of one 64-weight group; pos = 2i + (t>>1)):
//     (xh, xl of run t = 2(pos&1) elements 4i.., xh, xl of run t+1 ...)
// meta[u] (float4; Q4_K and Q6_K: two float4 per unit, meta[2u], meta[2u+1])
// holds the x-block scales and the sums s*(sum xh + sum xl/254) of the
// elements the unit covers, in the form each format's dot product uses.
//
// Round rd covers 8-element chunks gid = rd*TH + tid (TH threads per
// workgroup): x block blk = gid/4 (32 elements), elements 8*(gid%4) .. +7,
// so the four chunks of a block sit in one quad of lanes and the block's max
// and sums reduce with two quad-permute DPP steps.  x_round() loads one
// round (unconditionally: clamped address, value selected, so that no branch
// separates it from the weight loads that follow; the workgroup size is a
// compile-time constant for the same reason: blockDim is a memory load);
// quant_round() quantizes it.
template <int TH>
REALM_DEV void x_round(const float *__restrict__ x, int K, int U, int rd, float4 (&v)[2])
{
    const int gid = rd * TH + threadIdx.x;
    const int blk = gid >> 2, e0 = 8 * gid; // e0 = 32 blk + 8 (gid % 4)
    const bool live = blk < 2 * U && e0 < K; // K is a multiple of 32
    const float4 *p = reinterpret_cast<const float4 *>(x) + (min(e0, K - 8) >> 2);
    const float4 a = p[0], b = p[1], z = make_float4(0.f, 0.f, 0.f, 0.f);
    v[0] = live ? a : z;
    v[1] = live ? b : z;
}

REALM_DEV float quad_max(float v)
{
    v = fmaxf(v, dpp_f<0xB1, 0xF>(v)); // quad_perm [1,0,3,2]
    return fmaxf(v, dpp_f<0x4E, 0xF>(v)); // quad_perm [2,3,0,1]
}

REALM_DEV uint32_t pack_u8(float b0, float b1, float b2, float b3)
{
    uint32_t r = __builtin_amdgcn_cvt_pk_u8_f32(b0, 0, 0u);
    r = __builtin_amdgcn_cvt_pk_u8_f32(b1, 1, r);
    r = __builtin_amdgcn_cvt_pk_u8_f32(b2, 2, r);
    return __builtin_amdgcn_cvt_pk_u8_f32(b3, 3, r);
}

// A block whose values the int8 scaling cannot represent (a NaN or Inf, or
// a max |x| outside [EXACT_LO, EXACT_HI]) sets *flag: the token's rows are
// then recomputed on the exact f32 path (exact.h).
template <int FMT, int TH>
REALM_DEV void quant_round(int4 *rec, float4 *meta, int *flag, const float4 (&v)[2], int U,
                           int rd)
{
    const int gid = rd * TH + threadIdx.x;
    const int blk = gid >> 2, part = gid & 3;
    const bool live = blk < 2 * U;
    const float xs[8] = {v[0].x, v[0].y, v[0].z, v[0].w, v[1].x, v[1].y, v[1].z, v[1].w};
    float amax = 0.f;
    bool nonfinite = false;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        amax = fmaxf(amax, fabsf(xs[e]));
        nonfinite = nonfinite || !__builtin_isfinite(xs[e]);
    }
    amax = quad_max(amax);
    if (live && exact_needed(amax, nonfinite))
        *flag = 1;
    const float s = amax * (1.f / 127.f);
    const float inv = amax > 0.f ? 127.f / amax : 0.f;
    const float inv2 = 254.f * inv;
    // xh = round(x/s) in [-127, 127]; xl = round((x - s xh) 254/s) in
    // [-127, 127]; both biased by 128 into bytes, then xor 0x80 -> int8
    // in biased form: hb = xh + 128 = rint(x inv + 128) and
    // lb = xl + 128 = rint(x inv2 - 254 xh + 128) = rint(x inv2 + 32640 - 254 hb);
    // |x inv - xh| <= 1/2 keeps |xl| <= 127
    float hb[8], lb[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        hb[e] = rintf(fmaf(xs[e], inv, 128.f));
        lb[e] = rintf(fmaf(-254.f, hb[e], fmaf(xs[e], inv2, 32640.f)));
    }
    const uint32_t dh0 = pack_u8(hb[0], hb[1], hb[2], hb[3]) ^ 0x80808080u;
    const uint32_t dh1 = pack_u8(hb[4], hb[5], hb[6], hb[7]) ^ 0x80808080u;
    const uint32_t dl0 = pack_u8(lb[0], lb[1], lb[2], lb[3]) ^ 0x80808080u;
    const uint32_t dl1 = pack_u8(lb[4], lb[5], lb[6], lb[7]) ^ 0x80808080u;
    const int sh = dot4(dh1, 0x01010101u, dot4(dh0, 0x01010101u, 0));
    const int sl = dot4(dl1, 0x01010101u, dot4(dl0, 0x01010101u, 0));
    float part_sum = s * ((float)sh + (float)sl * (1.f / 254.f)); // 8 elements
    part_sum += dpp_f<0xB1, 0xF>(part_sum);                       // 16 elements
    if (FMT != FMT_Q6K)
        part_sum += dpp_f<0x4E, 0xF>(part_sum); // the whole block of 32
    if (!live)
        return;
    if (FMT == FMT_Q6K) {
        // x block blk of the 256-block B: h6 = (blk%8)/4, run t = blk%4; the
        // chunk lies in 16-run is = part/2 at dword positions 2(part%2) + k
        const int B = blk >> 3, h6 = (blk >> 2) & 1, t = blk & 3;
        const int is = part >> 1, i0 = 2 * (part & 1);
        const int u = 4 * B + 2 * h6 + is;
        int2 *r0 = reinterpret_cast<int2 *>(&rec[(2 * i0 + (t >> 1)) * U + u]) + (t & 1);
        int2 *r1 = reinterpret_cast<int2 *>(&rec[(2 * (i0 + 1) + (t >> 1)) * U + u]) + (t & 1);
        *r0 = make_int2((int)dh0, (int)dl0);
        *r1 = make_int2((int)dh1, (int)dl1);
        if ((part & 1) == 0) {
            float *m = reinterpret_cast<float *>(&meta[2 * u]);
            m[t] = s;            // scale of run t
            m[4 + t] = part_sum; // sum over the run's 16 elements
        }
    } else {
        const int u = blk >> 1, half = blk & 1;
        int2 *r0 = reinterpret_cast<int2 *>(&rec[(2 * part) * U + u]) + half;
        int2 *r1 = reinterpret_cast<int2 *>(&rec[(2 * part + 1) * U + u]) + half;
        *r0 = make_int2((int)dh0, (int)dl0);
        *r1 = make_int2((int)dh1, (int)dl1);
        if (part == 0) {
            if (FMT == FMT_Q4K) {
                // (s_a/254, s_b/(254*16), Sx_a, Sx_b), (8 Sx_b, ...): the
                // high-nibble dot products carry a factor 16 and a -8 offset
                float *m = reinterpret_cast<float *>(&meta[2 * u]);
                m[half] = s * (half ? 1.f / (254.f * 16.f) : 1.f / 254.f);
                m[2 + half] = part_sum;
                if (half)
                    m[4] = 8.f * part_sum;
            } else {
                float *m = reinterpret_cast<float *>(&meta[u]);
                m[half] = s;
                m[2 + half] = part_sum;
            }
        }
    }
}

// Per-format weight registers of one (row, unit) and their loader.  A pass
// reads each stream at a wave-uniform row base (scalar registers) plus a
// per-lane byte offset fixed for the whole kernel (the lane's row slot and
// unit), so the loads take the SGPR-base + 32-bit VGPR-offset form and no
// per-pass vector address arithmetic is needed.
struct Bases {
    const uint8_t *b0, *b1, *b2;
};

template <int FMT>
struct Unit;

// Q4_K: two 16-byte qs planes of the unit + the 16-byte block header.
template <>
struct Unit<FMT_Q4K> {
    uint4 q0, q1, hd;
    struct Off {
        uint32_t q, h;
    };
    // row strides (bytes) of the hdr and qs streams
    static __device__ __forceinline__ Off offsets(int slot, int u, int U)
    {
        return {(uint32_t)(slot * U * 32 + u * 16), (uint32_t)(slot * U * 4 + (u >> 2) * 16)};
    }
    static __device__ __forceinline__ size_t stride0(int U) { return (size_t)U * 4; }
    static __device__ __forceinline__ size_t stride1(int U) { return (size_t)U * 32; }
    static __device__ __forceinline__ size_t stride2(int) { return 0; }
    __device__ __forceinline__ void load(const Bases &b, const Off &o, int U)
    {
        q0 = ldg16(b.b1 + o.q);
        q1 = ldg16(b.b1 + o.q + (uint32_t)(U * 16));
        hd = ldg16(b.b0 + o.h);
    }
};

// Q6_K: three 16-byte quant planes, the unit's 4 sub-scales, the block's d.
template <>
struct Unit<FMT_Q6K> {
    uint4 qa, qb, qh;
    uint32_t sc, d;
    struct Off {
        uint32_t q, s, d;
    };
    static __device__ __forceinline__ Off offsets(int slot, int u, int U)
    {
        return {(uint32_t)(slot * U * 48 + u * 16),
                (uint32_t)(slot * U * 4 + (u >> 2) * 16 + (u & 3) * 4),
                (uint32_t)(slot * (U / 2) + (u >> 2) * 2)};
    }
    static __device__ __forceinline__ size_t stride0(int U) { return (size_t)(U / 2); }
    static __device__ __forceinline__ size_t stride1(int U) { return (size_t)U * 4; }
    static __device__ __forceinline__ size_t stride2(int U) { return (size_t)U * 48; }
    __device__ __forceinline__ void load(const Bases &b, const Off &o, int U)
    {
        qa = ldg16(b.b2 + o.q);
        qb = ldg16(b.b2 + o.q + (uint32_t)(U * 16));
        qh = ldg16(b.b2 + o.q + (uint32_t)(U * 32));
        sc = ldg4(b.b1 + o.s);
        d = *reinterpret_cast<const uint16_t *>(b.b0 + o.d);
    }
};

// Q8_0 (rows padded to KP = 64 U): four 16-byte planes and the two f16
// scales of the unit's blocks.
template <>
struct Unit<FMT_Q80> {
    uint4 q[4];
    uint32_t d;
    struct Off {
        uint32_t q, d;
    };
    static __device__ __forceinline__ Off offsets(int slot, int u, int U)
    {
        return {(uint32_t)(slot * U * 64 + u * 16), (uint32_t)(slot * U * 4 + u * 4)};
    }
    static __device__ __forceinline__ size_t stride0(int U) { return (size_t)U * 4; }
    static __device__ __forceinline__ size_t stride1(int U) { return (size_t)U * 64; }
    static __device__ __forceinline__ size_t stride2(int) { return 0; }
    __device__ __forceinline__ void load(const Bases &b, const Off &o, int U)
    {
#pragma unroll
        for (int c = 0; c < 4; ++c)
            q[c] = ldg16(b.b1 + o.q + (uint32_t)(c * U * 16));
        d = ldg4(b.b0 + o.d);
    }
};

// The reference's 32-element formats (quant.rs:10-70, 226-370), each
// element q' s + delta with a small integer q' (Q4_0/Q4_1: nibble - 8,
// Q5_0/Q5_1: 5-bit value - 16, Q8_1: int8), repacked at registration into
// the Q8_0 layout plus a delta stream (zero for Q4_0 and Q5_0): the Q8_0
// unit and the two f16 deltas of its blocks.
template <>
struct Unit<FMT_Q8M> {
    uint4 q[4];
    uint32_t d, m;
    struct Off {
        uint32_t q, d;
    };
    static __device__ __forceinline__ Off offsets(int slot, int u, int U)
    {
        return {(uint32_t)(slot * U * 64 + u * 16), (uint32_t)(slot * U * 4 + u * 4)};
    }
    static __device__ __forceinline__ size_t stride0(int U) { return (size_t)U * 4; }
    static __device__ __forceinline__ size_t stride1(int U) { return (size_t)U * 64; }
    static __device__ __forceinline__ size_t stride2(int U) { return (size_t)U * 4; }
    __device__ __forceinline__ void load(const Bases &b, const Off &o, int U)
    {
#pragma unroll
        for (int c = 0; c < 4; ++c)
            q[c] = ldg16(b.b1 + o.q + (uint32_t)(c * U * 16));
        d = ldg4(b.b0 + o.d);
        m = ldg4(b.b2 + o.d);
    }
};

REALM_DEV float combine(int ph, int pl, float s)
{
    return s * ((float)ph + (float)pl * (1.f / 254.f));
}

// Partial dot products of one row's unit with NT tokens' x.  xr(t, i) is
// token t's x record at dword position i (0..7) of the unit, xm(t, j) its
// metadata float4 j (Q4_K / Q6_K: 0, 1; Q8_0: 0): read from LDS, or from
// registers that hold them for the whole kernel.  The tokens go one after
// another with a scheduling barrier between them: left free, the compiler
// hoists every token's LDS records ahead of the first dot product (32
// VGPRs per token) and the multi-token kernels spill.
template <int FMT, int NT, class XR, class XM>
REALM_DEV void unit_dot(const Unit<FMT> &w, const XR &xr, const XM &xm, int u, int nan_fb,
                        float (&acc)[NT])
{
    if constexpr (FMT == FMT_Q4K) {
        const int g = u & 3;
        const float d = fix_scale(f16_bits_to_f32(w.hd.x), 0.00000006f, nan_fb);
        const float dm = fix_scale(f16_bits_to_f32(w.hd.x >> 16), 0.00000024f, nan_fb);
        const uint32_t pr = q4k_dev_pair(w.hd.y, w.hd.z, w.hd.w, g);
        const float sa = (float)(pr & 63u), ma = (float)((pr >> 6) & 63u);
        const float sb = (float)((pr >> 12) & 63u), mb = (float)((pr >> 18) & 63u);
        // low nibbles (sub-block 2g) read as int8 q in 0..15, high nibbles
        // (sub-block 2g+1, stored XOR 8) masked as int8 16 (q - 8); unpacked
        // once for all tokens
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t q = word(i < 4 ? w.q0 : w.q1, i & 3);
            lo[i] = q & 0x0F0F0F0Fu;
            hi[i] = q & 0xF0F0F0F0u;
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (t > 0)
                __builtin_amdgcn_sched_barrier(0);
            int ha = 0, la = 0, hb = 0, lb = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int4 xq = xr(t, i);
                ha = dot4(lo[i], (uint32_t)xq.x, ha);
                la = dot4(lo[i], (uint32_t)xq.y, la);
                hb = dot4(hi[i], (uint32_t)xq.z, hb);
                lb = dot4(hi[i], (uint32_t)xq.w, lb);
            }
            // (s_a/254, s_b/(254*16), Sx_a, Sx_b), (8 Sx_b, -, -, -)
            const float4 m = xm(t, 0), m2 = xm(t, 1);
            // exact integers: |ha*254 + la| < 2^24, |hb*254 + lb| < 2^28
            const float fa = (float)(ha * 254 + la);
            const float fb = (float)(hb * 254 + lb);
            const float ta = m.x * fa;            // sum over sub-block a of q * x
            const float tb = fmaf(m.y, fb, m2.x); // sum over b of (q - 8) x + 8 sum x
            acc[t] += d * fmaf(sa, ta, sb * tb) - dm * fmaf(ma, m.z, mb * m.w);
        }
    } else if constexpr (FMT == FMT_Q6K) {
        const float d = fix_scale(f16_bits_to_f32(w.d), 0.00000006f, nan_fb);
        // the 6-bit quants of the unit's four 16-runs, unpacked once for all
        // tokens: v[i][r] holds 4 quants of run r
        uint32_t v[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t a = word(w.qa, i), b = word(w.qb, i), h = word(w.qh, i);
            v[i][0] = (a & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
            v[i][1] = (b & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
            v[i][2] = ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
            v[i][3] = ((b >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (t > 0)
                __builtin_amdgcn_sched_barrier(0);
            int ph[4] = {0, 0, 0, 0}, pl[4] = {0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int4 x01 = xr(t, 2 * i), x23 = xr(t, 2 * i + 1);
                ph[0] = dot4(v[i][0], (uint32_t)x01.x, ph[0]);
                pl[0] = dot4(v[i][0], (uint32_t)x01.y, pl[0]);
                ph[1] = dot4(v[i][1], (uint32_t)x01.z, ph[1]);
                pl[1] = dot4(v[i][1], (uint32_t)x01.w, pl[1]);
                ph[2] = dot4(v[i][2], (uint32_t)x23.x, ph[2]);
                pl[2] = dot4(v[i][2], (uint32_t)x23.y, pl[2]);
                ph[3] = dot4(v[i][3], (uint32_t)x23.z, ph[3]);
                pl[3] = dot4(v[i][3], (uint32_t)x23.w, pl[3]);
            }
            // run scales, run sums
            const float4 ms = xm(t, 0), mx = xm(t, 1);
            const float sr[4] = {ms.x, ms.y, ms.z, ms.w}, sx[4] = {mx.x, mx.y, mx.z, mx.w};
            float part = 0.f;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                part += (float)(int8_t)(w.sc >> (8 * r)) *
                        (combine(ph[r], pl[r], sr[r]) - 32.f * sx[r]);
            acc[t] += d * part;
        }
    } else {
        const float da = f16_bits_to_f32(w.d), db = f16_bits_to_f32(w.d >> 16);
        float ma = 0.f, mb = 0.f;
        if constexpr (FMT == FMT_Q8M) {
            ma = f16_bits_to_f32(w.m);
            mb = f16_bits_to_f32(w.m >> 16);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (t > 0)
                __builtin_amdgcn_sched_barrier(0);
            int ha = 0, la = 0, hb = 0, lb = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int4 xq = xr(t, i);
                const uint32_t qa = word(w.q[i >> 2], i & 3);
                const uint32_t qb = word(w.q[2 + (i >> 2)], i & 3);
                ha = dot4(qa, (uint32_t)xq.x, ha);
                la = dot4(qa, (uint32_t)xq.y, la);
                hb = dot4(qb, (uint32_t)xq.z, hb);
                lb = dot4(qb, (uint32_t)xq.w, lb);
            }
            const float4 m = xm(t, 0);
            acc[t] += da * combine(ha, la, m.x) + db * combine(hb, lb, m.y);
            if constexpr (FMT == FMT_Q8M) // sum of (q' s + delta) x: + delta * sum x per block
                acc[t] += fmaf(ma, m.z, mb * m.w);
        }
    }
}


// One launch: NM matrices (1, or up to REALM_GEMV_MAX_MATS with NM = 4)
// that share x, rows concatenated, and NT tokens (a.m of them live: 1..NT;
// x is [m][K], each matrix's y is [m][its rows]).  LPR lanes share a row
// (64/LPR row slots per wave and pass), lane l owns units l, l+LPR, ...
// (UPL of them), and each wave keeps a ring of D passes in flight.  Every
// weight a lane loads is used for all NT tokens; token t's quantized x is
// the LDS region of TS = 10 U int4 starting at t TS (8 U records, then up
// to 2 U metadata float4).
// The fused pre-steps of the one-token "_n" / "_s" kernels (GemvArgs):
// element k of x' from the inputs, in the operation order of realm_rms_norm
// ((x + r) * inv * w) and realm_swiglu (g * (1 / (1 + exp(-g))) * u), so a
// fused product sees the values the separate launches would have written.
#define PRE_NONE 0
#define PRE_NORM 1
#define PRE_SWIGLU 2
REALM_DEV float4 pre_swiglu(float4 g, float4 u)
{
    return make_float4(g.x * (1.f / (1.f + expf(-g.x))) * u.x, g.y * (1.f / (1.f + expf(-g.y))) * u.y,
                       g.z * (1.f / (1.f + expf(-g.z))) * u.z, g.w * (1.f / (1.f + expf(-g.w))) * u.w);
}
REALM_DEV float4 pre_norm(float4 v, float inv, float4 w)
{
    return make_float4(v.x * inv * w.x, v.y * inv * w.y, v.z * inv * w.z, v.w * inv * w.w);
}
REALM_DEV float4 f4add(float4 a, float4 b)
{
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// exact_dot over x' of a fused kernel (the exact f32 path of a flagged row)
template <int FMT, int PRE>
REALM_DEV float exact_dot_pre(const void *w0, const void *w1, const void *w2, int row, int K,
                              int KX, const float *x, const float *pa, const float *pw, float inv,
                              int nan_fb, int k0, int step)
{
#pragma clang fp contract(off)
    float acc = 0.f;
    for (int k = k0; k < K; k += step) {
        float v;
        if constexpr (PRE == PRE_NORM) {
            const float h = pa ? x[k] + pa[k] : x[k];
            v = h * inv * pw[k];
        } else {
            const float g = x[k];
            v = g * (1.f / (1.f + expf(-g))) * pa[k];
        }
        acc += dev_weight<FMT>((const uint8_t *)w0, (const uint8_t *)w1, (const uint8_t *)w2, row,
                               k, KX, nan_fb) *
               v;
    }
    return acc;
}

template <int FMT, int LPR, int UPL, int D, int XR, int TH, int NM, int NT, int PRE = PRE_NONE>
REALM_DEV void gemv(const GemvArgs &a)
{
    static_assert(PRE == PRE_NONE || NT == 1, "the fused pre-steps are one-token kernels");
    using W = Unit<FMT>;
    extern __shared__ int4 lds[];
    const int K = a.K, KX = a.KX;
    const int U = KX >> 6;
    const int TS = 10 * U;
    int4 *rec = lds;
    float4 *meta = reinterpret_cast<float4 *>(lds + 8 * U);
    // per token: set when a block of its x needs the exact path
    int *xflag = reinterpret_cast<int *>(lds + NT * TS);
    const int M = NT == 1 ? 1 : a.m;
    // x of the lane's unit held in registers (one unit per lane, NT > 1)
    constexpr bool XREG = UPL == 1 && NT > 1;
    int4 xreg[XREG ? NT : 1][8];
    float4 mreg[XREG ? NT : 1][2];
    const int lane = threadIdx.x & 63;
    const int slot = lane / LPR, l = lane % LPR;
    constexpr int wpb = TH / 64;
    constexpr int RPP = 64 / LPR; // rows per pass
    // wave-uniform bookkeeping stays in scalar registers
    const int gw = __builtin_amdgcn_readfirstlane(blockIdx.x * wpb + (threadIdx.x >> 6));
    const int nw = gridDim.x * wpb;
    const int rs1 = a.row_start[1], rs2 = a.row_start[2], rs3 = a.row_start[3];
    const int rows = a.row_start[NM == 1 ? 1 : REALM_GEMV_MAX_MATS];
    const void *const w0[4] = {a.w0[0], a.w0[1], a.w0[2], a.w0[3]};
    const void *const w1[4] = {a.w1[0], a.w1[1], a.w1[2], a.w1[3]};
    const void *const w2[4] = {a.w2[0], a.w2[1], a.w2[2], a.w2[3]};
    float *const yv[4] = {a.y[0], a.y[1], a.y[2], a.y[3]};
    const float *const xp = a.x;
    const int nan_fb = a.nan_fb;
    int xbad = 0; // bit t: token t's x needs the exact path (set after staging)
    float pre_inv = 0.f; // _n: 1 / sqrt(mean((x + r)^2) + eps) (workgroup-uniform)
    // Every kernel argument is read here, in one batch of scalar loads ahead
    // of the first vector load (one statement, so all are live at once):
    // left alone, the compiler sinks some of these loads next to their uses,
    // and each batch is a round trip to the argument buffer on the kernel's
    // critical path.
    if constexpr (NM == 1)
        asm volatile("" ::"s"(K), "s"(KX), "s"(nw), "s"(rows), "s"(xp), "s"(nan_fb),
                     "s"(w0[0]), "s"(w1[0]), "s"(w2[0]), "s"(yv[0]), "s"(a.m));
    else
        asm volatile("" ::"s"(K), "s"(KX), "s"(nw), "s"(rs1), "s"(rs2), "s"(rs3), "s"(rows),
                     "s"(xp), "s"(nan_fb), "s"(w0[0]), "s"(w0[1]), "s"(w0[2]), "s"(w0[3]),
                     "s"(w1[0]), "s"(w1[1]), "s"(w1[2]), "s"(w1[3]), "s"(w2[0]), "s"(w2[1]),
                     "s"(w2[2]), "s"(w2[3]), "s"(yv[0]), "s"(yv[1]), "s"(yv[2]), "s"(yv[3]),
                     "s"(a.m));
    const int npass = (rows + RPP - 1) / RPP;
    // this wave's passes: p = gw + i*nw for i < T
    const int T = gw < npass ? (npass - gw + nw - 1) / nw : 0;

    // per-lane offsets, fixed for the kernel (a unit past the row end is
    // clamped to the last unit and masked in finish)
    typename W::Off off[UPL];
#pragma unroll
    for (int j = 0; j < UPL; ++j)
        off[j] = W::offsets(slot, min(l + j * LPR, U - 1), U);

    // Row base of pass i of this wave.  Pass indices past the wave's last
    // pass (ring slots with nothing left to do) re-read the wave's last
    // pass, whose lines were just fetched (no HBM traffic), so no load is
    // ever conditional; a wave with no pass at all reads the matrix's last
    // pass.  Every pass read is < npass, so with the 4 padding rows every
    // address stays inside the allocation.
    const int p_last = T > 0 ? gw + (T - 1) * nw : npass - 1;
    auto bases = [&](int i) {
        const int p = i < T ? gw + i * nw : p_last;
        const int row0 = p * RPP;
        int m = 0, lr = row0;
        if constexpr (NM > 1) {
            m = (row0 >= rs1 ? 1 : 0) + (row0 >= rs2 ? 1 : 0) + (row0 >= rs3 ? 1 : 0);
            lr = row0 - (m == 0 ? 0 : (m == 1 ? rs1 : (m == 2 ? rs2 : rs3)));
        }
        auto pick = [&](const void *const(&v)[4]) {
            if constexpr (NM == 1)
                return (const uint8_t *)v[0];
            else
                return (const uint8_t *)(m == 0 ? v[0] : (m == 1 ? v[1] : (m == 2 ? v[2] : v[3])));
        };
        return Bases{pick(w0) + (size_t)lr * W::stride0(U), pick(w1) + (size_t)lr * W::stride1(U),
                     pick(w2) + (size_t)lr * W::stride2(U)};
    };
    auto load_pass = [&](W(&w)[UPL], int i) {
        const Bases b = bases(i);
#pragma unroll
        for (int j = 0; j < UPL; ++j)
            w[j].load(b, off[j], U);
    };
    auto finish = [&](W(&w)[UPL], int i) {
        // With several units per lane the x records the loop reuses are
        // kept in registers but the per-unit scales and sums are re-read
        // from LDS every pass (an opaque zero offset stops the compiler from
        // hoisting them), which keeps a two-pass ring within the budget.
        const float4 *mt = meta;
        if constexpr (UPL >= 2) {
            uint32_t zero = 0;
            asm volatile("" : "+v"(zero));
            mt = meta + zero;
        }
        float acc[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t)
            acc[t] = 0.f;
#pragma unroll
        for (int j = 0; j < UPL; ++j) {
            const int u = l + j * LPR, uc = min(u, U - 1);
            float part[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t)
                part[t] = 0.f;
            if constexpr (XREG) {
                auto xr = [&](int t, int p) { return xreg[t][p]; };
                auto xm = [&](int t, int q) { return mreg[t][q]; };
                unit_dot<FMT, NT>(w[j], xr, xm, uc, nan_fb, part);
            } else {
                auto xr = [&](int t, int p) { return rec[t * TS + p * U + uc]; };
                auto xm = [&](int t, int q) {
                    return mt[t * TS + (ONE_META(FMT) ? uc : 2 * uc + q)];
                };
                unit_dot<FMT, NT>(w[j], xr, xm, uc, nan_fb, part);
            }
#pragma unroll
            for (int t = 0; t < NT; ++t)
                acc[t] += u < U ? part[t] : 0.f;
        }
        float v[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t)
            v[t] = group_total<LPR>(acc[t]);
        const int row = (gw + i * nw) * RPP + slot;
        if (__builtin_expect(xbad != 0, 0)) {
            // tokens flagged while staging x: the row on the exact f32 path,
            // K split over the row's LPR lanes (a padding row reads the last
            // row and is not stored)
            const int rc = min(row, rows - 1);
            int m = 0, lr = rc;
            if constexpr (NM > 1) {
                m = (rc >= rs1 ? 1 : 0) + (rc >= rs2 ? 1 : 0) + (rc >= rs3 ? 1 : 0);
                lr = rc - (m == 0 ? 0 : (m == 1 ? rs1 : (m == 2 ? rs2 : rs3)));
            }
            const void *e0 = m == 0 ? w0[0] : (m == 1 ? w0[1] : (m == 2 ? w0[2] : w0[3]));
            const void *e1 = m == 0 ? w1[0] : (m == 1 ? w1[1] : (m == 2 ? w1[2] : w1[3]));
            const void *e2 = m == 0 ? w2[0] : (m == 1 ? w2[1] : (m == 2 ? w2[2] : w2[3]));
#pragma unroll
            for (int t = 0; t < NT; ++t)
                if ((xbad >> t) & 1) {
                    if constexpr (PRE == PRE_NONE)
                        v[t] = group_total<LPR>(exact_dot<FMT>(e0, e1, e2, lr, K, KX,
                                                               xp + (size_t)min(t, M - 1) * K, 0,
                                                               nan_fb, l, LPR));
                    else
                        v[t] = group_total<LPR>(exact_dot_pre<FMT, PRE>(
                            e0, e1, e2, lr, K, KX, xp, a.pre_a, a.pre_w, pre_inv, nan_fb, l, LPR));
                }
        }
        if (l == LPR - 1 && row < rows) {
            float *y = yv[0];
            int lr = row, nrow = rows;
            if constexpr (NM > 1) {
                const int m = (row >= rs1 ? 1 : 0) + (row >= rs2 ? 1 : 0) + (row >= rs3 ? 1 : 0);
                const int r0 = m == 0 ? 0 : (m == 1 ? rs1 : (m == 2 ? rs2 : rs3));
                const int r1 = m == 0 ? rs1 : (m == 1 ? rs2 : (m == 2 ? rs3 : rows));
                y = m == 0 ? yv[0] : (m == 1 ? yv[1] : (m == 2 ? yv[2] : yv[3]));
                lr = row - r0;
                nrow = r1 - r0;
            }
#pragma unroll
            for (int t = 0; t < NT; ++t)
                if (t < M)
                    y[(size_t)t * nrow + lr] = v[t];
        }
    };

    // Prologue: x loads first (waiting for x then does not wait for
    // weights), then the first ring slot, then x is quantized into LDS while
    // those weights are in flight.
    const int rounds = (8 * U + TH - 1) / TH;
    // rounds held in registers per token (the register budget is shared
    // among the tokens)
    constexpr int XH = NT == 1 ? XR : (XR / NT > 0 ? XR / NT : 1);
    float4 xv[NT][XH][2];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int rd = 0; rd < XH; ++rd)
            x_round<TH>(xp + (size_t)min(t, M - 1) * K, K, U, rd, xv[t][rd]);
    // the fused pre-step's other inputs (residual or up; the norm weight),
    // loaded with x (the host only fuses a norm whose rounds all fit XH)
    constexpr int PXH = PRE == PRE_NONE ? 1 : XH;
    float4 pav[PXH][2], pwv[PXH][2];
    if constexpr (PRE != PRE_NONE) {
#pragma unroll
        for (int rd = 0; rd < XH; ++rd) {
            if (PRE == PRE_SWIGLU || a.pre_a)
                x_round<TH>(a.pre_a, K, U, rd, pav[rd]);
            if (PRE == PRE_NORM)
                x_round<TH>(a.pre_w, K, U, rd, pwv[rd]);
        }
    }
    if (threadIdx.x < NT)
        xflag[threadIdx.x] = 0;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    // Every wave of the workgroup issues its x loads before any wave issues
    // a weight load: the CU's vector memory path returns data in request
    // order, so x requests queued behind other waves' weight requests would
    // hold up the quantization (and the barrier) by a full weight fetch.
    // (The barrier also orders the flag reset above before any flag write.)
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    __builtin_amdgcn_sched_barrier(0);
    W w[D][UPL];
    load_pass(w[0], 0);
    if constexpr (PRE == PRE_SWIGLU) {
#pragma unroll
        for (int rd = 0; rd < XH; ++rd)
#pragma unroll
            for (int c = 0; c < 2; ++c)
                xv[0][rd][c] = pre_swiglu(xv[0][rd][c], pav[rd][c]);
    } else if constexpr (PRE == PRE_NORM) {
        // h = x + r (written out once, by workgroup 0), its sum of squares
        // over the workgroup (every workgroup the same), then h inv w
        float ss = 0.f;
#pragma unroll
        for (int rd = 0; rd < XH; ++rd) {
            const int e0 = 8 * (rd * TH + (int)threadIdx.x);
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                float4 hv = xv[0][rd][c];
                if (a.pre_a)
                    hv = f4add(hv, pav[rd][c]);
                xv[0][rd][c] = hv;
                ss += hv.x * hv.x + hv.y * hv.y + hv.z * hv.z + hv.w * hv.w;
            }
            if (a.pre_sum && blockIdx.x == 0 && rd < rounds && e0 < K) {
                float4 *o = reinterpret_cast<float4 *>(a.pre_sum + e0);
                o[0] = xv[0][rd][0];
                o[1] = xv[0][rd][1];
            }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1)
            ss += __shfl_xor(ss, off, 64);
        __shared__ float pre_red[TH / 64];
        if ((threadIdx.x & 63) == 0)
            pre_red[threadIdx.x >> 6] = ss;
        lds_barrier();
        float total = 0.f;
#pragma unroll
        for (int wv = 0; wv < TH / 64; ++wv)
            total += pre_red[wv];
        pre_inv = 1.f / sqrtf(total / (float)K + a.pre_eps);
#pragma unroll
        for (int rd = 0; rd < XH; ++rd)
#pragma unroll
            for (int c = 0; c < 2; ++c)
                xv[0][rd][c] = pre_norm(xv[0][rd][c], pre_inv, pwv[rd][c]);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int rd = 0; rd < XH; ++rd)
            if (rd < rounds)
                quant_round<FMT, TH>(rec + t * TS, meta + t * TS, xflag + t, xv[t][rd], U, rd);
#pragma unroll
    for (int t = 0; t < NT; ++t)
        for (int rd = XH; rd < rounds; ++rd) {
            float4 v[2];
            x_round<TH>(xp + (size_t)min(t, M - 1) * K, K, U, rd, v);
            if constexpr (PRE == PRE_SWIGLU) { // (a fused norm has no rounds here)
                float4 u[2];
                x_round<TH>(a.pre_a, K, U, rd, u);
                v[0] = pre_swiglu(v[0], u[0]);
                v[1] = pre_swiglu(v[1], u[1]);
            }
            quant_round<FMT, TH>(rec + t * TS, meta + t * TS, xflag + t, v, U, rd);
        }
    lds_barrier();
    // bit t: token t takes the exact path (wave-uniform)
    int xbad_v = 0;
#pragma unroll
    for (int t = 0; t < NT; ++t)
        xbad_v |= (xflag[t] != 0 ? 1 : 0) << t;
    xbad = __builtin_amdgcn_readfirstlane(xbad_v);
    // One unit per lane, several tokens: the lane's unit is the same in
    // every pass, so its records and metadata of every token move to
    // registers once (re-reading them from LDS each pass would take NT x
    // 160 bytes of LDS bandwidth per lane and pass, more than the CU's LDS
    // delivers at the weight stream's rate).
    if constexpr (XREG) {
        const int uc = min(l, U - 1);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
#pragma unroll
            for (int p = 0; p < 8; ++p)
                xreg[t][p] = rec[t * TS + p * U + uc];
#pragma unroll
            for (int q = 0; q < 2; ++q)
                mreg[t][q] = meta[t * TS + (ONE_META(FMT) ? uc : 2 * uc + q)];
        }
    }
    // The rest of the ring is issued only now: a larger burst ahead of the
    // x staging would delay x (same memory queues) and so the first pass.
#pragma unroll
    for (int s = 1; s < D; ++s)
        load_pass(w[s], s);

    // Every load is unconditional on the path that reaches it and every
    // path into a join carries the same D slots in flight, so each wait the
    // compiler places is for exactly the slot about to be used.
    int i = 0;
    for (; i + D < T; i += D) {
#pragma unroll
        for (int s = 0; s < D; ++s) {
            finish(w[s], i + s);
            load_pass(w[s], i + s + D);
        }
    }
#pragma unroll
    for (int s = 0; s < D; ++s) {
        if (i + s >= T)
            break;
        finish(w[s], i + s);
    }
}

} // namespace

// x rounds held in registers across the prologue: all of them for the
// longest row a variant serves (64 * UPL units, 8 chunks of 8 elements
// each), at most 8 (further rounds are loaded after the weights)
#define GEMV_XR(UPL, TH) ((512 * (UPL) + (TH) - 1) / (TH) < 8 ? (512 * (UPL) + (TH) - 1) / (TH) : 8)
// Workgroup size by units per lane and ring depth: 1024 threads (<= 128
// VGPRs) for one unit per lane and up to 4 passes in flight, fewer threads
// and more registers beyond.
#define GEMV_TH(UPL, D)                                                                    \
    ((UPL) == 1 ? ((D) <= 4 ? 1024 : 512)                                                    \
                : ((UPL) <= 3 ? ((D) == 1 ? 1024 : ((UPL) == 2 || (D) == 2 ? 512 : 256)) : 256))

// Workgroup size of the multi-token kernels: with one unit per lane the x
// of every token stays in registers (40 VGPRs per token), so 512 or 256
// threads; beyond, the per-token sums and the longer dot product body need
// more registers per ring slot, so halved where the one-token size would
// spill.
#define GEMV_THN(UPL, D, NT)                                                                  \
    ((NT) == 1 ? GEMV_TH(UPL, D)                                                              \
               : ((UPL) == 1 ? ((NT) == 2 || (D) <= 3 ? 512 : 256)                            \
                             : ((UPL) == 2 ? ((D) == 1 && (NT) == 2 ? 1024 : 512)               \
                                           : ((UPL) == 3 && (D) == 1 ? 512 : 256))))

// Variant: lanes per row, units per lane, ring depth, matrices (1 or 4),
// tokens (the one-token kernels carry no token suffix).
#define DEF_GEMV1P(NAME, FMT, LPR, UPL, D, NM, NT, SUF, PRE)                                 \
    extern "C" __global__ __launch_bounds__(GEMV_THN(UPL, D, NT)) void                       \
        realm_gemv_##NAME##_l##LPR##_u##UPL##_d##D##_m##NM##SUF(GemvArgs a)                  \
    {                                                                                        \
        gemv<FMT, LPR, UPL, D, GEMV_XR(UPL, GEMV_THN(UPL, D, NT)), GEMV_THN(UPL, D, NT), NM,  \
             NT, PRE>(a);                                                                     \
    }
#define DEF_GEMV1(NAME, FMT, LPR, UPL, D, NM, NT, SUF)                                       \
    DEF_GEMV1P(NAME, FMT, LPR, UPL, D, NM, NT, SUF, PRE_NONE)
#if REALM_GEMV_FMT == FMT_Q4K
#define DEF_GEMV2(LPR, UPL, D, NM, NT, SUF) DEF_GEMV1(q4k, FMT_Q4K, LPR, UPL, D, NM, NT, SUF)
#define DEF_GEMVP(LPR, UPL, D, NM, SUF, PRE) DEF_GEMV1P(q4k, FMT_Q4K, LPR, UPL, D, NM, 1, SUF, PRE)
#elif REALM_GEMV_FMT == FMT_Q6K
#define DEF_GEMV2(LPR, UPL, D, NM, NT, SUF) DEF_GEMV1(q6k, FMT_Q6K, LPR, UPL, D, NM, NT, SUF)
#define DEF_GEMVP(LPR, UPL, D, NM, SUF, PRE) DEF_GEMV1P(q6k, FMT_Q6K, LPR, UPL, D, NM, 1, SUF, PRE)
#elif REALM_GEMV_FMT == FMT_Q80
#define DEF_GEMV2(LPR, UPL, D, NM, NT, SUF) DEF_GEMV1(q80, FMT_Q80, LPR, UPL, D, NM, NT, SUF)
#define DEF_GEMVP(LPR, UPL, D, NM, SUF, PRE) DEF_GEMV1P(q80, FMT_Q80, LPR, UPL, D, NM, 1, SUF, PRE)
#else
#define DEF_GEMV2(LPR, UPL, D, NM, NT, SUF) DEF_GEMV1(q8m, FMT_Q8M, LPR, UPL, D, NM, NT, SUF)
#endif

#if defined(REALM_GEMV_PRE)
// The decoder layer's fused one-token kernels: "_n" (RMSNorm before the
// product; grouped Q/K/V and gate/up, NM = 4) and "_s" (SwiGLU; W_down,
// NM = 1), in the ring depths the host picks for them (1-3 for one unit per
// lane, 1-2 for two or three, 1 beyond).
#define DEF_GEMV_PRE(LPR, UPL, D) DEF_GEMVP(LPR, UPL, D, 4, _n, PRE_NORM) DEF_GEMVP(LPR, UPL, D, 1, _s, PRE_SWIGLU)
DEF_GEMV_PRE(16, 1, 1) DEF_GEMV_PRE(16, 1, 2) DEF_GEMV_PRE(16, 1, 3)
DEF_GEMV_PRE(32, 1, 1) DEF_GEMV_PRE(32, 1, 2) DEF_GEMV_PRE(32, 1, 3)
DEF_GEMV_PRE(64, 1, 1) DEF_GEMV_PRE(64, 1, 2) DEF_GEMV_PRE(64, 1, 3)
DEF_GEMV_PRE(64, 2, 1) DEF_GEMV_PRE(64, 2, 2)
DEF_GEMV_PRE(64, 3, 1) DEF_GEMV_PRE(64, 3, 2)
DEF_GEMV_PRE(64, 4, 1) DEF_GEMV_PRE(64, 5, 1) DEF_GEMV_PRE(64, 6, 1) DEF_GEMV_PRE(64, 7, 1)
DEF_GEMV_PRE(64, 8, 1)
#elif !defined(REALM_GEMV_NT) || REALM_GEMV_NT == 1
#define DEF_GEMV(LPR, UPL, D) DEF_GEMV2(LPR, UPL, D, 1, 1, ) DEF_GEMV2(LPR, UPL, D, 4, 1, )

// The one-token variants the host chooses from (ring depths per
// units-per-lane must match the host's tables).
#define DEF_GEMV_ONE_UNIT(LPR)                                                                \
    DEF_GEMV(LPR, 1, 1) DEF_GEMV(LPR, 1, 2) DEF_GEMV(LPR, 1, 3) DEF_GEMV(LPR, 1, 4)           \
        DEF_GEMV(LPR, 1, 6) DEF_GEMV(LPR, 1, 8) DEF_GEMV(LPR, 1, 12)
DEF_GEMV_ONE_UNIT(16)
DEF_GEMV_ONE_UNIT(32)
DEF_GEMV_ONE_UNIT(64)
DEF_GEMV(64, 2, 1)
DEF_GEMV(64, 2, 2)
DEF_GEMV(64, 2, 3)
DEF_GEMV(64, 2, 4)
DEF_GEMV(64, 3, 1)
DEF_GEMV(64, 3, 2)
DEF_GEMV(64, 3, 3)
DEF_GEMV(64, 3, 4)
DEF_GEMV(64, 3, 6)
DEF_GEMV(64, 4, 1)
DEF_GEMV(64, 4, 2)
DEF_GEMV(64, 5, 1)
DEF_GEMV(64, 5, 2)
DEF_GEMV(64, 6, 1)
DEF_GEMV(64, 7, 1)
DEF_GEMV(64, 8, 1)
#else
// Multi-token variants (2 or 4 tokens; 3 tokens run the 4-token kernels):
// ring depths 1-4 for one unit per lane, 1-2 for two or three, 1 beyond
// (each pass carries NT times the dot products, so deeper rings gain less).
#define DEF_GEMV_NT(LPR, UPL, D, NT, SUF)                                                     \
    DEF_GEMV2(LPR, UPL, D, 1, NT, SUF) DEF_GEMV2(LPR, UPL, D, 4, NT, SUF)
#define DEF_GEMV_TOKENS(NT, SUF)                                                              \
    DEF_GEMV_NT(16, 1, 1, NT, SUF) DEF_GEMV_NT(16, 1, 2, NT, SUF)                             \
    DEF_GEMV_NT(16, 1, 3, NT, SUF) DEF_GEMV_NT(16, 1, 4, NT, SUF)                             \
    DEF_GEMV_NT(32, 1, 1, NT, SUF) DEF_GEMV_NT(32, 1, 2, NT, SUF)                             \
    DEF_GEMV_NT(32, 1, 3, NT, SUF) DEF_GEMV_NT(32, 1, 4, NT, SUF)                             \
    DEF_GEMV_NT(64, 1, 1, NT, SUF) DEF_GEMV_NT(64, 1, 2, NT, SUF)                             \
    DEF_GEMV_NT(64, 1, 3, NT, SUF) DEF_GEMV_NT(64, 1, 4, NT, SUF)                             \
    DEF_GEMV_NT(64, 2, 1, NT, SUF) DEF_GEMV_NT(64, 2, 2, NT, SUF)                             \
    DEF_GEMV_NT(64, 3, 1, NT, SUF) DEF_GEMV_NT(64, 3, 2, NT, SUF)                             \
    DEF_GEMV_NT(64, 4, 1, NT, SUF) DEF_GEMV_NT(64, 5, 1, NT, SUF)                             \
    DEF_GEMV_NT(64, 6, 1, NT, SUF) DEF_GEMV_NT(64, 7, 1, NT, SUF)                             \
    DEF_GEMV_NT(64, 8, 1, NT, SUF)
#if REALM_GEMV_NT == 2
DEF_GEMV_TOKENS(2, _t2)
#elif REALM_GEMV_NT == 4
DEF_GEMV_TOKENS(4, _t4)
#else
#error "REALM_GEMV_NT must be 1, 2 or 4"
#endif
#endif

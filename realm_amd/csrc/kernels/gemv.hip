// Decode GEMV, one token: y[n] = sum_k W[n,k] x[k] for resident Q4_K / Q6_K /
// Q8_0 weights in the device layout of common.h, up to 4 matrices that share
// x per launch (rows concatenated: e.g. Q/K/V, or gate/up).
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
// handles 64/LPR row slots of R rows per pass.  The grid is persistent: each
// wave strides over passes and keeps two in flight (the next pass's weights
// load while the current one computes).  Quantized x lives in LDS as one
// 16-byte record per (unit, dword position), laid out [position][unit], so
// lanes of a wave read consecutive records (no bank conflicts).
#include "common.h"
#include "kernel_args.h"

using namespace realm;
using realm::GemvArgs;

#define FMT_Q4K 0
#define FMT_Q6K 1
#define FMT_Q80 2

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

// Max over aligned groups of 8 lanes (one x block of 32 = 8 x float4) and sum
// over aligned groups of 4 (one 16-element half block).
REALM_DEV float max8(float v)
{
    v = fmaxf(v, __shfl_xor(v, 1, 64));
    v = fmaxf(v, __shfl_xor(v, 2, 64));
    return fmaxf(v, __shfl_xor(v, 4, 64));
}
REALM_DEV int sum4i(int v)
{
    v += __shfl_xor(v, 1, 64);
    return v + __shfl_xor(v, 2, 64);
}

REALM_DEV uint32_t pack4(int a, int b, int c, int d)
{
    return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16) |
           ((uint32_t)(d & 0xFF) << 24);
}

// Quantize x into LDS.  rec[pos * U + u] (int4) holds, for unit u and dword
// position pos, the xh and xl dwords its dot products need:
//   Q4_K / Q8_0 (unit = x blocks 2u, 2u+1; pos = i in 0..7):
//     (xh, xl of block 2u elements 4i..4i+3, xh, xl of block 2u+1 elements 4i..)
//   Q6_K (unit = 16-runs t = 0..3 of one 64-weight group; pos = 2i + (t>>1)):
//     (xh, xl of run t = 2(pos&1) elements 4i.., xh, xl of run t+1 ...)
// meta[u] (float4; Q6_K: two float4 per unit) holds the x-block scales and
// the sums s*(sum xh + sum xl/254) of the elements the unit covers.
//
// Round rd covers 4-element chunks gid = rd*TH + tid (TH threads per
// workgroup), i.e. x block gid/8, chunk gid%8.  x_round() loads one round;
// quant_round() quantizes it.  The load is unconditional (clamped address,
// value selected) so that no branch separates it from the weight loads that
// follow: the workgroup size is a compile-time constant for the same reason
// (blockDim is a memory load).
template <int TH>
REALM_DEV float4 x_round(const float *__restrict__ x, int K, int U, int rd)
{
    const int gid = rd * TH + threadIdx.x;
    const int blk = gid >> 3, c8 = gid & 7;
    const int e0 = 32 * blk + 4 * c8;
    const float4 v = reinterpret_cast<const float4 *>(x)[min(e0, K - 4) >> 2];
    return (blk < 2 * U && e0 < K) ? v : make_float4(0.f, 0.f, 0.f, 0.f);
}

template <int FMT, int TH>
REALM_DEV void quant_round(int4 *rec, float4 *meta, float4 v, int U, int rd)
{
    const int gid = rd * TH + threadIdx.x;
    const int blk = gid >> 3, c8 = gid & 7;
    const bool live = blk < 2 * U;
    float amax = max8(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    const float s = amax * (1.f / 127.f);
    const float inv = amax > 0.f ? 127.f / amax : 0.f;
    const float inv2 = amax > 0.f ? 254.f * 127.f / amax : 0.f;
    const float xs[4] = {v.x, v.y, v.z, v.w};
    int h[4], lo[4], sh = 0, sl = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        h[e] = (int)rintf(xs[e] * inv);
        lo[e] = max(-127, min(127, (int)rintf((xs[e] - s * (float)h[e]) * inv2)));
        sh += h[e];
        sl += lo[e];
    }
    sh = sum4i(sh);
    sl = sum4i(sl);
    const float part = s * ((float)sh + (float)sl * (1.f / 254.f)); // 16 elements
    const float other = __shfl_xor(part, 4, 64);                      // the other half
    if (!live)
        return;
    const uint32_t dh = pack4(h[0], h[1], h[2], h[3]);
    const uint32_t dl = pack4(lo[0], lo[1], lo[2], lo[3]);
    if (FMT == FMT_Q6K) {
        // x block blk of the 256-block B: h6 = (blk%8)/4, run t = blk%4; the
        // chunk lies in 16-run is = c8/4 at dword position i = c8%4
        const int B = blk >> 3, h6 = (blk >> 2) & 1, t = blk & 3;
        const int is = c8 >> 2, i = c8 & 3;
        const int u = 4 * B + 2 * h6 + is;
        int *r = reinterpret_cast<int *>(&rec[(2 * i + (t >> 1)) * U + u]);
        r[2 * (t & 1)] = (int)dh;
        r[2 * (t & 1) + 1] = (int)dl;
        if (i == 0) {
            float *m = reinterpret_cast<float *>(&meta[2 * u]);
            m[t] = s;        // scale of run t
            m[4 + t] = part; // sum over the run's 16 elements
        }
    } else {
        const int u = blk >> 1, half = blk & 1, i = c8;
        int *r = reinterpret_cast<int *>(&rec[i * U + u]);
        r[2 * half] = (int)dh;
        r[2 * half + 1] = (int)dl;
        if (c8 == 0) {
            float *m = reinterpret_cast<float *>(&meta[u]);
            m[half] = s;
            m[2 + half] = part + other; // whole block of 32
        }
    }
}

// Scale/min pair for sub-blocks 2g and 2g+1 from header dwords s0,s1,s2
// (crates/realm-core/src/quant.rs:110-122) with g known only at run time.
REALM_DEV void q4k_pair_rt(uint32_t s0, uint32_t s1, uint32_t s2, int g, float &sc_lo,
                           float &m_lo, float &sc_hi, float &m_hi)
{
    int sh = 16 * (g & 1); // byte 2g&3 of a dword
    uint32_t a0 = s0 >> sh, a1 = s1 >> sh, a2 = s2 >> sh;
    uint32_t sl, ml, shh, mh;
    if (g < 2) {
        sl = a0 & 63u;
        ml = a1 & 63u;
        shh = (a0 >> 8) & 63u;
        mh = (a1 >> 8) & 63u;
    } else {
        sl = (a2 & 0xFu) | (((a0 >> 6) & 3u) << 4);
        ml = ((a2 >> 4) & 0xFu) | (((a1 >> 6) & 3u) << 4);
        shh = ((a2 >> 8) & 0xFu) | (((a0 >> 14) & 3u) << 4);
        mh = ((a2 >> 12) & 0xFu) | (((a1 >> 14) & 3u) << 4);
    }
    sc_lo = (float)sl;
    m_lo = (float)ml;
    sc_hi = (float)shh;
    m_hi = (float)mh;
}

// Per-format weight registers of one (row, unit) and their loader.
template <int FMT>
struct Unit;

template <>
struct Unit<FMT_Q4K> {
    uint4 q0, q1, hd;
    __device__ __forceinline__ void load(const uint8_t *w0, const uint8_t *w1, const uint8_t *,
                                         size_t row, int u, int K)
    {
        const size_t U = (size_t)(K >> 6);
        const uint8_t *qp = w1 + row * (U * 32) + 16 * u;
        q0 = ldg16(qp);          // plane 0
        q1 = ldg16(qp + U * 16); // plane 1
        hd = ldg16(w0 + (row * (size_t)(K >> 8) + (u >> 2)) * 16);
    }
    __device__ __forceinline__ void zero() { q0 = q1 = hd = make_uint4(0, 0, 0, 0); }
};

template <>
struct Unit<FMT_Q6K> {
    uint4 qa, qb, qh;
    uint32_t sc, d;
    __device__ __forceinline__ void load(const uint8_t *w0, const uint8_t *w1, const uint8_t *w2,
                                         size_t row, int u, int K)
    {
        size_t B = (size_t)(K >> 8), U = 4 * B;
        const uint8_t *qp = w2 + row * (U * 48) + 16 * u;
        qa = ldg16(qp);
        qb = ldg16(qp + U * 16);
        qh = ldg16(qp + U * 32);
        size_t blk = row * B + (u >> 2);
        sc = ldg4(w1 + blk * 16 + 4 * (u & 3));
        d = *reinterpret_cast<const uint16_t *>(w0 + blk * 2);
    }
    __device__ __forceinline__ void zero()
    {
        qa = qb = qh = make_uint4(0, 0, 0, 0);
        sc = d = 0;
    }
};

template <>
struct Unit<FMT_Q80> {
    uint4 q[4];
    uint32_t d;
    // K here is the padded row length Kp
    __device__ __forceinline__ void load(const uint8_t *w0, const uint8_t *w1, const uint8_t *,
                                         size_t row, int u, int KP)
    {
        const size_t U = (size_t)(KP >> 6);
        const uint8_t *qp = w1 + row * (size_t)KP + 16 * u;
#pragma unroll
        for (int c = 0; c < 4; ++c)
            q[c] = ldg16(qp + c * (U * 16));
        d = ldg4(w0 + (row * (size_t)(KP >> 5) + 2 * u) * 2);
    }
    __device__ __forceinline__ void zero()
    {
#pragma unroll
        for (int c = 0; c < 4; ++c)
            q[c] = make_uint4(0, 0, 0, 0);
        d = 0;
    }
};

REALM_DEV float combine(int ph, int pl, float s)
{
    return s * ((float)ph + (float)pl * (1.f / 254.f));
}

// Partial dot products of R rows with one unit of x.
template <int FMT, int R>
REALM_DEV void unit_dot(const Unit<FMT> (&w)[R], const int4 *rec, const float4 *meta, int U,
                        int u, int nan_fb, float (&acc)[R])
{
    if constexpr (FMT == FMT_Q4K) {
        int hl[R], ll[R], hh[R], lh[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
            hl[r] = ll[r] = hh[r] = lh[r] = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int4 xq = rec[i * U + u];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                uint32_t q = word(i < 4 ? w[r].q0 : w[r].q1, i & 3);
                uint32_t lo = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu;
                hl[r] = dot4(lo, (uint32_t)xq.x, hl[r]);
                ll[r] = dot4(lo, (uint32_t)xq.y, ll[r]);
                hh[r] = dot4(hi, (uint32_t)xq.z, hh[r]);
                lh[r] = dot4(hi, (uint32_t)xq.w, lh[r]);
            }
        }
        const float4 m = meta[u]; // (s_lo, s_hi, sum_lo, sum_hi)
        const int g = u & 3;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float d = fix_scale(f16_bits_to_f32(w[r].hd.x), 0.00000006f, nan_fb);
            float dm = fix_scale(f16_bits_to_f32(w[r].hd.x >> 16), 0.00000024f, nan_fb);
            float sl, ml, sh, mh;
            q4k_pair_rt(w[r].hd.y, w[r].hd.z, w[r].hd.w, g, sl, ml, sh, mh);
            acc[r] += d * (sl * combine(hl[r], ll[r], m.x) + sh * combine(hh[r], lh[r], m.y)) -
                      dm * (ml * m.z + mh * m.w);
        }
    } else if constexpr (FMT == FMT_Q6K) {
        int ph[R][4], pl[R][4];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int t = 0; t < 4; ++t)
                ph[r][t] = pl[r][t] = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int4 x01 = rec[(2 * i) * U + u], x23 = rec[(2 * i + 1) * U + u];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                uint32_t a = word(w[r].qa, i), b = word(w[r].qb, i), h = word(w[r].qh, i);
                uint32_t v0 = (a & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
                uint32_t v1 = (b & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
                uint32_t v2 = ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
                uint32_t v3 = ((b >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
                ph[r][0] = dot4(v0, (uint32_t)x01.x, ph[r][0]);
                pl[r][0] = dot4(v0, (uint32_t)x01.y, pl[r][0]);
                ph[r][1] = dot4(v1, (uint32_t)x01.z, ph[r][1]);
                pl[r][1] = dot4(v1, (uint32_t)x01.w, pl[r][1]);
                ph[r][2] = dot4(v2, (uint32_t)x23.x, ph[r][2]);
                pl[r][2] = dot4(v2, (uint32_t)x23.y, pl[r][2]);
                ph[r][3] = dot4(v3, (uint32_t)x23.z, ph[r][3]);
                pl[r][3] = dot4(v3, (uint32_t)x23.w, pl[r][3]);
            }
        }
        const float4 ms = meta[2 * u], mx = meta[2 * u + 1]; // run scales, run sums
        const float s[4] = {ms.x, ms.y, ms.z, ms.w}, sx[4] = {mx.x, mx.y, mx.z, mx.w};
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float d = fix_scale(f16_bits_to_f32(w[r].d), 0.00000006f, nan_fb);
            float part = 0.f;
#pragma unroll
            for (int t = 0; t < 4; ++t)
                part += (float)(int8_t)(w[r].sc >> (8 * t)) *
                        (combine(ph[r][t], pl[r][t], s[t]) - 32.f * sx[t]);
            acc[r] += d * part;
        }
    } else {
        int ha[R], la[R], hb[R], lb[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
            ha[r] = la[r] = hb[r] = lb[r] = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int4 xq = rec[i * U + u];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                uint32_t qa = word(w[r].q[i >> 2], i & 3);
                uint32_t qb = word(w[r].q[2 + (i >> 2)], i & 3);
                ha[r] = dot4(qa, (uint32_t)xq.x, ha[r]);
                la[r] = dot4(qa, (uint32_t)xq.y, la[r]);
                hb[r] = dot4(qb, (uint32_t)xq.z, hb[r]);
                lb[r] = dot4(qb, (uint32_t)xq.w, lb[r]);
            }
        }
        const float4 m = meta[u];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float da = f16_bits_to_f32(w[r].d), db = f16_bits_to_f32(w[r].d >> 16);
            acc[r] += da * combine(ha[r], la[r], m.x) + db * combine(hb[r], lb[r], m.y);
        }
    }
}


template <int FMT, int LPR, int UPL, int R, int XR, int TH>
REALM_DEV void gemv(const GemvArgs &a)
{
    extern __shared__ int4 lds[];
    const int K = a.K, KX = a.KX;
    const int U = KX >> 6;
    int4 *rec = lds;
    float4 *meta = reinterpret_cast<float4 *>(lds + 8 * U);
    const int lane = threadIdx.x & 63;
    const int slot = lane / LPR, l = lane % LPR;
    constexpr int wpb = TH / 64;
    // wave-uniform: keeps pass/row/matrix bookkeeping (and the kernarg
    // pointer tables) in scalar registers, out of the vector memory queue
    const int gw = __builtin_amdgcn_readfirstlane(blockIdx.x * wpb + (threadIdx.x >> 6));
    const int nw = gridDim.x * wpb;
    constexpr int RPP = (64 / LPR) * R; // rows per pass per wave
    const int rs1 = a.row_start[1], rs2 = a.row_start[2], rs3 = a.row_start[3];
    const int rows = a.row_start[REALM_GEMV_MAX_MATS];
    const void *const w0[4] = {a.w0[0], a.w0[1], a.w0[2], a.w0[3]};
    const void *const w1[4] = {a.w1[0], a.w1[1], a.w1[2], a.w1[3]};
    const void *const w2[4] = {a.w2[0], a.w2[1], a.w2[2], a.w2[3]};
    float *const yv[4] = {a.y[0], a.y[1], a.y[2], a.y[3]};
    const float *const xp = a.x;
    const int nan_fb = a.nan_fb;
    // Every kernel argument is read here, in one batch of scalar loads ahead
    // of the first vector load.  Left alone, the compiler sinks some of these
    // loads next to their uses, behind the x loads, and each such batch is a
    // round trip to the argument buffer on the kernel's critical path.
    // (one statement, so that all of them are live at once)
    asm volatile("" ::"s"(K), "s"(KX), "s"(nw), "s"(rs1), "s"(rs2), "s"(rs3), "s"(rows),
                 "s"(xp), "s"(nan_fb), "s"(w0[0]), "s"(w0[1]), "s"(w0[2]), "s"(w0[3]),
                 "s"(w1[0]), "s"(w1[1]), "s"(w1[2]), "s"(w1[3]), "s"(w2[0]), "s"(w2[1]),
                 "s"(w2[2]), "s"(w2[3]), "s"(yv[0]), "s"(yv[1]), "s"(yv[2]), "s"(yv[3]),
                 "s"(a.pad));
    const int npass = (rows + RPP - 1) / RPP;
    const int wk = FMT == FMT_Q80 ? KX : K; // row length of the quant stream

    // matrix of a global row; pointer choice by selects, never by indexing
    // the kernarg arrays with a per-lane value
    auto mat_of = [&](int row) {
        return (row >= rs1 ? 1 : 0) + (row >= rs2 ? 1 : 0) + (row >= rs3 ? 1 : 0);
    };
    auto pick = [](int m, auto v0, auto v1, auto v2, auto v3) {
        return m == 0 ? v0 : (m == 1 ? v1 : (m == 2 ? v2 : v3));
    };
    // No branch writes the registers of an in-flight load (a branch makes the
    // compiler wait for every outstanding load): a row past the end is
    // clamped to the last row and a unit past the end to the last unit; the
    // results of both are masked in finish.
    auto load_pass = [&](Unit<FMT>(&w)[UPL][R], int p) {
        const int r0 = p * RPP + slot * R;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = min(r0 + r, rows - 1);
            const int m = mat_of(row);
            const size_t lr = (size_t)(row - pick(m, 0, rs1, rs2, rs3));
            const uint8_t *p0 = (const uint8_t *)pick(m, w0[0], w0[1], w0[2], w0[3]);
            const uint8_t *p1 = (const uint8_t *)pick(m, w1[0], w1[1], w1[2], w1[3]);
            const uint8_t *p2 = (const uint8_t *)pick(m, w2[0], w2[1], w2[2], w2[3]);
#pragma unroll
            for (int j = 0; j < UPL; ++j)
                w[j][r].load(p0, p1, p2, lr, min(l + j * LPR, U - 1), wk);
        }
    };
    auto finish = [&](Unit<FMT>(&w)[UPL][R], int pp) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
            acc[r] = 0.f;
#pragma unroll
        for (int j = 0; j < UPL; ++j) {
            const int u = l + j * LPR;
            float part[R];
#pragma unroll
            for (int r = 0; r < R; ++r)
                part[r] = 0.f;
            unit_dot<FMT, R>(w[j], rec, meta, U, min(u, U - 1), nan_fb, part);
#pragma unroll
            for (int r = 0; r < R; ++r)
                acc[r] += u < U ? part[r] : 0.f;
        }
        const int r0 = pp * RPP + slot * R;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float v = group_total<LPR>(acc[r]);
            const int row = r0 + r;
            if (l == LPR - 1 && row < rows) {
                const int m = mat_of(row);
                float *y = pick(m, yv[0], yv[1], yv[2], yv[3]);
                y[row - pick(m, 0, rs1, rs2, rs3)] = v;
            }
        }
    };

    // Prologue: x loads first (so waiting for x does not wait for weights),
    // then the weights of the wave's first two passes, then x is quantized
    // into LDS while those loads are in flight.
    const int rounds = (16 * U + TH - 1) / TH;
    float4 xv[XR];
#pragma unroll
    for (int rd = 0; rd < XR; ++rd)
        xv[rd] = x_round<TH>(xp, K, U, rd);
    Unit<FMT> A[UPL][R], B[UPL][R];
    int p = gw;
    load_pass(A, p);
    load_pass(B, p + nw);
#pragma unroll
    for (int rd = 0; rd < XR; ++rd)
        if (rd < rounds)
            quant_round<FMT, TH>(rec, meta, xv[rd], U, rd);
    for (int rd = XR; rd < rounds; ++rd)
        quant_round<FMT, TH>(rec, meta, x_round<TH>(xp, K, U, rd), U, rd);
    lds_barrier();

    // Two passes in flight per wave: each computes while the other loads.
    // The wave's passes are p = gw + i*nw, i < T.  Every load below is
    // unconditional on the path that reaches it and every path into a join
    // carries the same loads in flight (A then B), so each wait the compiler
    // places covers exactly the pass about to be used.  No load is issued
    // past the wave's last pass, except the prologue's B when T < 2 (the host
    // sizes the grid so that T >= 2 wherever the matrix allows it).
    int left = p < npass ? (npass - p + nw - 1) / nw : 0;
    for (;;) {
        if (left <= 2)
            break;
        finish(A, p);
        load_pass(A, p + 2 * nw);
        if (left == 3) {
            finish(B, p + nw);
            finish(A, p + 2 * nw);
            return;
        }
        finish(B, p + nw);
        load_pass(B, p + 3 * nw);
        p += 2 * nw;
        left -= 2;
    }
    if (left >= 1)
        finish(A, p);
    if (left >= 2)
        finish(B, p + nw);
}

} // namespace

// x rounds held in registers across the prologue: all of them for the
// longest row a variant serves (64 * UPL units, 16 float4 each)
#define GEMV_XR(UPL, TH) ((1024 * (UPL) + (TH) - 1) / (TH))

// Variant (lanes per row, units per lane, rows per pass, threads per
// workgroup).  The workgroup size is a compile-time constant: at most 1024
// threads (<= 128 VGPRs) while a lane owns one unit, fewer beyond.
#define DEF_GEMV1(NAME, FMT, LPR, UPL, R, TH)                                                 \
    extern "C" __global__ __launch_bounds__(TH) void                                         \
        realm_gemv_##NAME##_l##LPR##_u##UPL##_r##R##_t##TH(GemvArgs a)                       \
    {                                                                                        \
        gemv<FMT, LPR, UPL, R, GEMV_XR(UPL, TH), TH>(a);                                     \
    }
#define DEF_GEMV_T(LPR, UPL, R, TH)              \
    DEF_GEMV1(q4k, FMT_Q4K, LPR, UPL, R, TH)     \
    DEF_GEMV1(q6k, FMT_Q6K, LPR, UPL, R, TH)     \
    DEF_GEMV1(q80, FMT_Q80, LPR, UPL, R, TH)
#define DEF_GEMV(LPR, UPL, R)                                             \
    DEF_GEMV_T(LPR, UPL, R, 256)                                          \
    DEF_GEMV_T(LPR, UPL, R, 512)                                          \
    DEF_GEMV_T(LPR, UPL, R, 1024)
#define DEF_GEMV_MID(UPL) DEF_GEMV_T(64, UPL, 1, 256) DEF_GEMV_T(64, UPL, 1, 512)

// The variants the host chooses from.
DEF_GEMV(16, 1, 1)
DEF_GEMV(16, 1, 2)
DEF_GEMV(32, 1, 1)
DEF_GEMV(32, 1, 2)
DEF_GEMV(64, 1, 1)
DEF_GEMV(64, 1, 2)
DEF_GEMV_MID(2)
DEF_GEMV_MID(3)
DEF_GEMV_T(64, 4, 1, 256)
DEF_GEMV_T(64, 5, 1, 256)
DEF_GEMV_T(64, 6, 1, 256)
DEF_GEMV_T(64, 7, 1, 256)
DEF_GEMV_T(64, 8, 1, 256)

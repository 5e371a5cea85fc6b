// LDS-tiled batched GEMM for resident Q4_K / Q6_K / Q8_0 weights, for the
// batch sizes where activations are worth sharing between waves (batched
// decode of 16+ tokens, prefill):
//
//   Y[t][n] = sum_k X[t][k] W[n][k]      on v_mfma_f32_32x32x16_f16
//
// Operands and exactness as in gemm.hip (xprep's f16 hi/lo activations, here
// in slot order 1; weights decoded to sc*q, (q-32)*sc or q, exact in f16;
// block scales applied to f32 partial sums).  MFMA roles: A = activations
// (32 token slots x 16 k), B = weights (16 k x 32 rows).  Lane l = r32 + 32h
// supplies A[r32][(h, e)] and B[(h, e)][r32]; D lane l holds row r32 for
// token slots 8(v/4) + 4h + v%4, v < 16, so each lane scales its own row's
// sums with the block scale it decoded itself.
//
//  * A workgroup owns GROWS = WR*TN*32 rows x GTOK tokens (and, with a K
//    split, 1/KS of the 256-blocks).  WR x WT waves: wave (wr, wt) owns TN
//    32-row tiles and TM 32-slot token tiles.
//  * A block's activations (GTOK tokens x 256 k, the lo part too for f32
//    input) are staged once into LDS, double buffered: every wave reads its A
//    fragments from there.  The next block's activations are loaded into
//    registers while the current block is multiplied and written to the other
//    buffer afterwards: one barrier per block.
//  * A lane's weights (its row, 128 k of each block) are loaded a block ahead
//    into registers and decoded there.
//  * Tile order puts all token tiles (and K splits) of a row tile on one XCD
//    (workgroup id mod 8), where they share the row tile's weights in L2.
// Modes: p = f32 input packed as (hi, lo) slot pairs (16 tokens per tile),
// s = f32 input with a second MFMA on the lo part, b = bf16 input (hi only).
#include "mfma_common.h"
#include "kernel_args.h"

using namespace realm;

typedef float floatx16 __attribute__((ext_vector_type(16)));

namespace realm_tiled {

#define REALM_MEMBER __device__ __forceinline__

REALM_DEV floatx16 mfma32(half8_t a, half8_t b, floatx16 c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// One matrix of a launch: its weight streams and shape.
struct Mat {
    const void *w0, *w1, *w2;
    int N, K, KX;
};

// Raw weight bytes of one 32-row tile and one 256-k block as lane
// (r32 = row within the tile, h = lane half) needs them: k 128h .. 128h+127
// of the block (Q4_K, Q6_K), or (Q8_0) units 2(i&1) + h of plane i/2, i < 8.
template <int FMT>
struct Raw;
template <>
struct Raw<FMT_Q4K> {
    uint4 q[4]; // qs of units 2h + uu, plane p: q[2 uu + p]
    uint4 hd;   // block header
};
template <>
struct Raw<FMT_Q6K> {
    uint4 a[2], b[2], hq[2]; // planes of units 2h + is
    uint2 sc;                // the sub-block scales of those two units
    uint32_t d;              // f16 block scale (low half)
};
template <>
struct Raw<FMT_Q80> {
    uint4 q[8]; // load i: plane i/2 of unit 4 blk + 2(i&1) + h, k-steps 2i, 2i+1
    uint4 d;    // the eight f16 block scales
};

// Byte offsets of a lane's weights (its row, lane half h) in the weight
// streams, fixed for the kernel.  A block adds a workgroup-uniform amount, so
// every weight load is a scalar base plus this 32-bit offset (the host keeps
// tiled weights under 4 GB).  Rows past N read row N-1 (always resident);
// their results land in D columns that are never stored.
struct LaneOff {
    uint32_t o0, o1, o2;
};
template <int FMT>
REALM_DEV LaneOff lane_off(const Mat &g, int row, int h)
{
    const uint32_t r = (uint32_t)row;
    if constexpr (FMT == FMT_Q4K) // w0 header [row][blk] 16 B; w1 qs planes, K/2 B per row
        return {r * (uint32_t)(g.K >> 8) * 16u, r * (uint32_t)(g.K >> 1) + 32u * h, 0u};
    else if constexpr (FMT == FMT_Q6K) // w0 d [row][blk] 2 B; w1 sc 16 B; w2 planes, 3K/4 B
        return {r * (uint32_t)(g.K >> 8) * 2u, r * (uint32_t)(g.K >> 8) * 16u + 8u * h,
                r * (uint32_t)(g.K >> 6) * 48u + 32u * h};
    else // Q8_0: w0 d [row][KX/32] 2 B; w1 q planes, KX B per row
        return {r * (uint32_t)(g.KX >> 5) * 2u, r * (uint32_t)g.KX + 16u * h, 0u};
}

REALM_DEV void load_raw(Raw<FMT_Q4K> &r, const Mat &g, const LaneOff &o, int blk)
{
    const size_t U = (size_t)(g.K >> 6);
    const uint8_t *q0 = (const uint8_t *)g.w1 + (size_t)blk * 64, *q1 = q0 + U * 16;
    r.q[0] = ldg16(q0 + o.o1);
    r.q[1] = ldg16(q1 + o.o1);
    r.q[2] = ldg16(q0 + o.o1 + 16);
    r.q[3] = ldg16(q1 + o.o1 + 16);
    r.hd = ldg16((const uint8_t *)g.w0 + (size_t)blk * 16 + o.o0);
}
REALM_DEV void load_raw(Raw<FMT_Q6K> &r, const Mat &g, const LaneOff &o, int blk)
{
    const size_t U = (size_t)(g.K >> 6);
    const uint8_t *p0 = (const uint8_t *)g.w2 + (size_t)blk * 64, *p1 = p0 + U * 16,
                  *p2 = p0 + U * 32;
#pragma unroll
    for (int is = 0; is < 2; ++is) {
        r.a[is] = ldg16(p0 + o.o2 + 16 * is);
        r.b[is] = ldg16(p1 + o.o2 + 16 * is);
        r.hq[is] = ldg16(p2 + o.o2 + 16 * is);
    }
    r.sc = ldg8((const int8_t *)g.w1 + (size_t)blk * 16 + o.o1);
    r.d = *reinterpret_cast<const uint16_t *>((const uint8_t *)g.w0 + (size_t)blk * 2 + o.o0);
}
REALM_DEV void load_raw(Raw<FMT_Q80> &r, const Mat &g, const LaneOff &o, int blk)
{
    const size_t U = (size_t)(g.KX >> 6);
    const uint8_t *q = (const uint8_t *)g.w1 + (size_t)blk * 64;
#pragma unroll
    for (int i = 0; i < 8; ++i) // plane i/2 of unit 4 blk + 2(i&1) + h (h in o1)
        r.q[i] = ldg16(q + (i >> 1) * (U * 16) + (i & 1) * 32 + o.o1);
    r.d = ldg16((const uint8_t *)g.w0 + (size_t)blk * 16 + o.o0);
}

// Per-block decode of a Raw tile into B fragments of k-step s (0..15).
template <int FMT, bool WIDE>
struct Dec;

template <bool WIDE>
struct Dec<FMT_Q4K, WIDE> {
    uint32_t w[16];
    float d, dm;
    // sub-blocks 4h + e' (e' = 0..3): (sc, -1024 sc) for nibbles at bits 0..3
    // of a half word, (sc / 16, -64 sc) for nibbles at bits 4..7
    half2_t sc2[4], cc2[4], sd2[4], cd2[4];
    // -dmin * m of sub-blocks (4h, 4h+1), (4h+2, 4h+3) as f16 hi + lo: the
    // f32 product (at most 17 significant bits, a multiple of 2^-24) splits
    // exactly into two f16 for every finite dmin
    uint32_t mh[2], ml[2];
    REALM_MEMBER void init(const Raw<FMT_Q4K> &r, int h, int nan_fb)
    {
#pragma unroll
        for (int i = 0; i < 4; ++i) { // as stored: high nibbles XOR 8 (undone in frag)
            w[4 * i + 0] = r.q[i].x;
            w[4 * i + 1] = r.q[i].y;
            w[4 * i + 2] = r.q[i].z;
            w[4 * i + 3] = r.q[i].w;
        }
        d = fix_scale(f16_bits_to_f32(r.hd.x), 0.00000006f, nan_fb);
        dm = fix_scale(f16_bits_to_f32(r.hd.x >> 16), 0.00000024f, nan_fb);
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
            const uint32_t pr = q4k_dev_pair(r.hd.y, r.hd.z, r.hd.w, 2 * h + pp);
            const uint32_t s0 = pr & 63u, m0 = (pr >> 6) & 63u;
            const uint32_t s1 = (pr >> 12) & 63u, m1 = (pr >> 18) & 63u;
            sc2[2 * pp] = splat2((float)s0);
            cc2[2 * pp] = splat2(-1024.f * (float)s0);
            sd2[2 * pp] = splat2((float)s0 * 0.0625f);
            cd2[2 * pp] = splat2(-64.f * (float)s0);
            sc2[2 * pp + 1] = splat2((float)s1);
            cc2[2 * pp + 1] = splat2(-1024.f * (float)s1);
            sd2[2 * pp + 1] = splat2((float)s1 * 0.0625f);
            cd2[2 * pp + 1] = splat2(-64.f * (float)s1);
            const float v0 = -dm * (float)m0, v1 = -dm * (float)m1;
            const _Float16 h0 = (_Float16)v0, h1 = (_Float16)v1;
            half2_t hh = {h0, h1};
            half2_t ll = {(_Float16)(v0 - (float)h0), (_Float16)(v1 - (float)h1)};
            mh[pp] = u32(hh);
            ml[pp] = u32(ll);
        }
    }
    // qs dword s (unit 2h + s/8): low nibbles in sub-block 2(s/8), high in
    // 2(s/8) + 1.  A nibble at bits 0..3 of a half word, OR 0x6400, is the
    // f16 1024 + q: times sc minus 1024 sc gives sc q.  A nibble at bits 4..7
    // gives 1024 + 16 q: times sc / 16 minus 64 sc gives sc q.  Both exact.
    REALM_MEMBER half8_t frag(int s) const
    {
        const uint32_t x = w[s], y = x >> 8;
        const int sb = 2 * (s >> 3);
        // the masks live in VGPRs so that mask-and-merge is one v_and_or_b32
        // (VOP3 takes no literal, and one SGPR at most)
        uint32_t mlo = 0x000F000Fu, mhi = 0x00F000F0u, chi = 0x64806480u;
        __asm__("" : "+v"(mlo), "+v"(mhi), "+v"(chi));
        const uint32_t p0 = (x & mlo) | 0x64006400u; // bytes 0, 2 low nibbles
        const uint32_t p1 = (y & mlo) | 0x64006400u; // bytes 1, 3 low nibbles
        // high nibbles: bitop3 table 0x6A is mhi ? x ^ chi : chi, i.e. the
        // nibble with its stored XOR 8 undone (chi bit 7) merged into 0x6400
        const uint32_t p2 = __builtin_amdgcn_bitop3_b32(x, mhi, chi, 0x6A); // bytes 0, 2
        const uint32_t p3 = __builtin_amdgcn_bitop3_b32(y, mhi, chi, 0x6A); // bytes 1, 3
        return h8(u32(__builtin_elementwise_fma(h2(p0), sc2[sb], cc2[sb])),
                  u32(__builtin_elementwise_fma(h2(p1), sc2[sb], cc2[sb])),
                  u32(__builtin_elementwise_fma(h2(p2), sd2[sb + 1], cd2[sb + 1])),
                  u32(__builtin_elementwise_fma(h2(p3), sd2[sb + 1], cd2[sb + 1])));
    }
};

template <bool WIDE>
struct Dec<FMT_Q6K, WIDE> {
    uint32_t a[2][4], b[2][4], hq[2][4];
    float d;
    half2_t s2[2][4], s2h[2][4]; // [unit is][t]
    REALM_MEMBER void init(const Raw<FMT_Q6K> &r, int h, int nan_fb)
    {
#pragma unroll
        for (int is = 0; is < 2; ++is) {
            a[is][0] = r.a[is].x; a[is][1] = r.a[is].y; a[is][2] = r.a[is].z; a[is][3] = r.a[is].w;
            b[is][0] = r.b[is].x; b[is][1] = r.b[is].y; b[is][2] = r.b[is].z; b[is][3] = r.b[is].w;
            hq[is][0] = r.hq[is].x; hq[is][1] = r.hq[is].y; hq[is][2] = r.hq[is].z; hq[is][3] = r.hq[is].w;
            const uint32_t scw = is ? r.sc.y : r.sc.x;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int sc = (int)(int8_t)(scw >> (8 * t));
                if (WIDE) {
                    s2[is][t] = splat2((float)(sc & 15));
                    s2h[is][t] = splat2(16.f * (float)(sc >> 4));
                } else {
                    s2[is][t] = splat2((float)sc);
                }
            }
        }
        d = fix_scale(f16_bits_to_f32(r.d), 0.00000006f, nan_fb);
    }
    // (q - 32) of k-step s as f16 pairs, f16(1024 + q) - 1056: ql dword
    // (s/2)&3 of unit s/8, plane A (s even: t = 0 low nibbles, t = 2 high) or
    // B (s odd: t = 1, 3), with the qh bits of those t
    REALM_MEMBER void quads(int s, half2_t (&q)[4]) const
    {
        const int is = s >> 3, q4 = (s >> 1) & 3, tp = s & 1;
        const uint32_t src = tp ? b[is][q4] : a[is][q4];
        const uint32_t qd = hq[is][q4];
        const uint32_t vlo = (src & 0x0F0F0F0Fu) | (((qd >> (2 * tp)) & 0x03030303u) << 4);
        const uint32_t vhi = ((src >> 4) & 0x0F0F0F0Fu) | (((qd >> (2 * tp + 4)) & 0x03030303u) << 4);
        const half2_t off2 = splat2(-1056.f);
        q[0] = h2((vlo & 0x00FF00FFu) | 0x64006400u) + off2;
        q[1] = h2(((vlo >> 8) & 0x00FF00FFu) | 0x64006400u) + off2;
        q[2] = h2((vhi & 0x00FF00FFu) | 0x64006400u) + off2;
        q[3] = h2(((vhi >> 8) & 0x00FF00FFu) | 0x64006400u) + off2;
    }
};

template <bool WIDE>
struct Dec<FMT_Q80, WIDE> {}; // Q8_0 decodes straight from the raw bytes

// Eight Q8_0 quants as f16, in the order bytes 0, 2, 1, 3, 4, 6, 5, 7: each
// byte XOR 0x80 (u = q + 128) placed under 0x64 by one byte permute is the
// f16 1152 + q; minus 1152 gives q exactly.
REALM_DEV half8_t q80_frag(uint2 q)
{
    const half2_t off2 = splat2(-1152.f);
    const uint32_t ua = q.x ^ 0x80808080u, ub = q.y ^ 0x80808080u, c = 0x64646464u;
    // selector bytes 0-3 pick from the second operand, 4-7 from the first
    const half2_t q0 = h2(__builtin_amdgcn_perm(c, ua, 0x04020400u)) + off2;
    const half2_t q1 = h2(__builtin_amdgcn_perm(c, ua, 0x04030401u)) + off2;
    const half2_t q2 = h2(__builtin_amdgcn_perm(c, ub, 0x04020400u)) + off2;
    const half2_t q3 = h2(__builtin_amdgcn_perm(c, ub, 0x04030401u)) + off2;
    return h8(u32(q0), u32(q1), u32(q2), u32(q3));
}

// A Q8_0 k-step fragment with its block scale d folded in, as an exact f16
// pair: hi = RN(d q) and lo = d q - hi.  d q has at most 19 significant bits
// and is a multiple of ulp(d); hi is a multiple of ulp(d) too, so lo is a
// multiple of ulp(d) no larger than half an ulp of hi (at most 8 bits): the
// fused multiply-add computes it exactly.  hi is finite while |d| < 512
// (|q| <= 128); rows with a larger or non-finite scale are flagged
// (q80_big_scale) and take the exact f32 path.
REALM_DEV void q80_split(uint2 q, uint32_t d2bits, half8_t &hi, half8_t &lo)
{
#pragma clang fp contract(off)
    const uint4 u = __builtin_bit_cast(uint4, q80_frag(q));
    const uint32_t qv[4] = {u.x, u.y, u.z, u.w};
    const half2_t d2 = h2(d2bits);
    uint32_t hv[4], lv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const half2_t p = h2(qv[i]) * d2;
        hv[i] = u32(p);
        lv[i] = u32(__builtin_elementwise_fma(h2(qv[i]), d2, -p));
    }
    hi = h8(hv[0], hv[1], hv[2], hv[3]);
    lo = h8(lv[0], lv[1], lv[2], lv[3]);
}

// Nonzero when one of the two f16 scales in w has |d| >= 512 or is not
// finite ((bits & 0x7FFF) >= 0x6000, tested per half without carries).
REALM_DEV uint32_t q80_big_scale(uint32_t w)
{
    return ((w & 0x7FFF7FFFu) + 0x20002000u) & 0x80008000u;
}

REALM_DEV half8_t lds_h8(const uint8_t *p)
{
    return __builtin_bit_cast(half8_t, *reinterpret_cast<const uint4 *>(p));
}

} // namespace realm_tiled

using namespace realm_tiled;

#define MODE_P 0 // f32, (hi, lo) slot pairs
#define MODE_S 1 // f32, separate lo MFMA
#define MODE_B 2 // bf16, hi only

template <int FMT, int WR, int WT, int TN, int TM, int MODE, bool WIDE, int NS>
REALM_DEV void gemm_tiled(const GemmArgs &g)
{
    constexpr int NT = WR * WT * 64;
    constexpr bool PACK = MODE == MODE_P, SEP = MODE == MODE_S;
    constexpr int TOK = PACK ? 16 : 32;     // tokens per 32-slot tile
    constexpr int GROWS = WR * TN * 32;     // rows per workgroup
    constexpr int GTOK = WT * TM * TOK;     // tokens per workgroup
    constexpr int SROWS = WT * TM * 32;     // LDS slot rows per part
    constexpr int NPART = SEP ? 2 : 1;
    // Q8_0 and wide Q6_K run two MFMAs per k-step on two weight fragments
    // (Q8_0: the hi and lo parts of d q, summed straight into acc)
    constexpr bool TWO = WIDE || FMT == FMT_Q80;
    constexpr int RS = 528;                 // bytes per slot row: 256 f16 + 16 pad
    constexpr int MRS = 32;                 // bytes per Q4_K min-term row
    constexpr int XB = NPART * SROWS * RS;
    constexpr bool MIN = FMT == FMT_Q4K;
    constexpr int BUF = XB + (MIN ? SROWS * MRS : 0);
    // LDS image of one block, in 16-byte chunks: NPART parts of SROWS slot
    // rows of 33 chunks (32 of data, 1 of padding), then the Q4_K min rows
    // (2 chunks each).  It is written by direct-to-LDS loads: lane i of a
    // load instruction fills chunk 64n + i of the image.
    constexpr int XCHK = NPART * SROWS * (RS / 16); // activation chunks incl. padding
    constexpr int MCHK = MIN ? SROWS * 2 : 0;
    constexpr int XINS = (XCHK + 63) / 64, MINS = (MCHK + 63) / 64;
    constexpr int NW = WR * WT;
    constexpr int BUFB = (XINS + MINS) * 1024; // bytes written per buffer
    constexpr int MOFF = XINS * 1024;          // start of the min rows
    static_assert(BUFB >= BUF, "LDS image covers the buffer");
    __shared__ __attribute__((aligned(1024))) uint8_t lbuf[NS][BUFB];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wr = wave % WR, wt = wave / WR;
    const int r32 = lane & 31, h = lane >> 5;
    const int uwave = __builtin_amdgcn_readfirstlane(wave);

    // Tile order: workgroup L runs on XCD x = L mod 8.  The XCDs form an
    // XR x XT grid over (row tile, K split) x token tiles (XT = g.xt): XCD x
    // owns a contiguous block of both, so its L2 holds 1/XT of the
    // activations while its row tiles' weights stream through.  Workgroup ids
    // past an XCD's block exit at once.
    const int KS = g.ksplit, XT = g.xt, XR = 8 / XT;
    const int RT = g.rtiles;
    const int TT = (g.M + GTOK - 1) / GTOK;
    const int RK = RT * KS;
    const int RKX = (RK + XR - 1) / XR, TTX = (TT + XT - 1) / XT;
    const int L = blockIdx.x, xcd = L & 7, j = L >> 3;
    const int jr = j / TTX, jt = j - jr * TTX;
    const int rk = (xcd / XT) * RKX + jr, tt = (xcd % XT) * TTX + jt;
    if (jr >= RKX || rk >= RK || tt >= TT)
        return;
    const int kc = rk % KS, rt = rk / KS;
    // the matrix (segment) of row tile rt; selects, not an indexed array, so
    // that nothing lands in scratch memory
    const int seg = (rt >= g.seg_tile[1]) + (rt >= g.seg_tile[2]) + (rt >= g.seg_tile[3]);
    auto pick = [&](auto a0, auto a1, auto a2, auto a3) {
        return seg == 0 ? a0 : seg == 1 ? a1 : seg == 2 ? a2 : a3;
    };
    const Mat mat{pick(g.seg_w0[0], g.seg_w0[1], g.seg_w0[2], g.seg_w0[3]),
                  pick(g.seg_w1[0], g.seg_w1[1], g.seg_w1[2], g.seg_w1[3]),
                  pick(g.seg_w2[0], g.seg_w2[1], g.seg_w2[2], g.seg_w2[3]),
                  pick(g.seg_n[0], g.seg_n[1], g.seg_n[2], g.seg_n[3]), g.K, g.KX};
    float *const yseg = pick(g.seg_y[0], g.seg_y[1], g.seg_y[2], g.seg_y[3]);
    const int rtl = rt - pick(g.seg_tile[0], g.seg_tile[1], g.seg_tile[2], g.seg_tile[3]);
    const int m0 = tt * GTOK;
    const int row0 = rtl * GROWS + wr * TN * 32 + r32; // this lane's row in tile a: row0 + 32a
    const int nblk = (FMT == FMT_Q80 ? g.KX : g.K) >> 8;
    const int b0 = kc * nblk / KS, b1 = (kc + 1) * nblk / KS;

    const uint8_t *xh = (const uint8_t *)g.xh, *xl = (const uint8_t *)g.xl;
    const uint8_t *xm = (const uint8_t *)g.xm;
    const size_t xrow = (size_t)g.KX * 2;
    const size_t dxl = (size_t)(xl - xh); // lo part: a separate workspace (f32 input)
    typedef __attribute__((address_space(3))) void lds_void_t;
    typedef __attribute__((address_space(1))) const void gbl_void_t;
    // Source of this lane's chunk in direct-to-LDS load n of block 0; block
    // blk reads 512 bytes (activations) or 32 bytes (min rows) further on.
    auto dma_src = [&](int n) -> const uint8_t * {
        const uint8_t *src;
        if (n < XINS) {
            const int c = 64 * n + lane;
            int part = 0, cc = c;
            if (NPART == 2 && cc >= SROWS * (RS / 16)) {
                part = 1;
                cc -= SROWS * (RS / 16);
            }
            const int srow = cc / (RS / 16);
            int col = cc - srow * (RS / 16);
            const bool live = c < XCHK;
            col = col < 32 ? col : 0; // padding chunk: reload chunk 0 of its row
            int tok, lo;
            if (PACK) {
                tok = m0 + 16 * (srow >> 5) + ((srow & 31) >> 1);
                lo = srow & 1;
            } else {
                tok = m0 + srow;
                lo = part;
            }
            if (!live) { // past the image: reload the first row's chunk
                tok = m0;
                lo = 0;
                col = 0;
            }
            // xh or xl by arithmetic (a select of two pointers can become
            // a lookup through scratch memory)
            src = xh + (size_t)lo * dxl + (size_t)tok * xrow + col * 16;
        } else {
            const int c = 64 * (n - XINS) + lane;
            const int srow = c >> 1, hh = c & 1;
            // packed: a token's lo slot row reads token TT * GTOK, which
            // xprep leaves all zero
            int tok = PACK ? ((srow & 1) ? TT * GTOK : m0 + 16 * (srow >> 5) + ((srow & 31) >> 1))
                           : m0 + srow;
            if (c >= MCHK) // past the image
                tok = m0;
            src = xm + ((size_t)tok * nblk * 2 + hh) * 16;
        }
        return src;
    };
    constexpr int NDW = (XINS + MINS + NW - 1) / NW; // loads per wave and block
    const uint8_t *dsrc[NDW];
#pragma unroll
    for (int i = 0; i < NDW; ++i)
        dsrc[i] = dma_src(min(i * NW + uwave, XINS + MINS - 1));
    // issue this wave's share of the block's direct-to-LDS loads
    auto stage = [&](uint8_t *buf, int blk) {
#pragma unroll
        for (int i = 0; i < NDW; ++i) {
            const int n = i * NW + uwave;
            if (n < XINS + MINS)
                __builtin_amdgcn_global_load_lds((gbl_void_t *)(dsrc[i] + blk * (n < XINS ? 512 : 32)),
                                                 (lds_void_t *)(buf + 1024 * n), 16, 0, 0);
        }
    };

    auto zero16 = [](floatx16 &v) {
#pragma unroll
        for (int e = 0; e < 16; ++e)
            v[e] = 0.f;
    };
    floatx16 acc[TN][TM];
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
        for (int b = 0; b < TM; ++b)
            zero16(acc[a][b]);

    // One 256-block: MFMAs on the activations in buf, weights in wcur, while
    // the next block's weights load into wnxt and its activations into nbuf.
    // vector-memory instructions one stage issues in every wave (at least):
    // its share of the direct-to-LDS loads plus its weight loads
    constexpr int GMIN = (XINS + MINS) / NW + TN * (FMT == FMT_Q4K ? 5 : FMT == FMT_Q6K ? 8 : 9);
    // Q8_0: rows (lane's tile a) with a scale that d q in f16 cannot hold
    uint32_t bad[TN];
#pragma unroll
    for (int a = 0; a < TN; ++a)
        bad[a] = 0u;
    // wait until at most k stages' loads are in flight (k < NS - 1), i.e.
    // everything issued before them has landed
    auto wait_stages = [&](int k) {
        if (NS > 3 && k >= 2)
            __builtin_amdgcn_s_waitcnt(0x0F70 | ((2 * GMIN) & 15) | (((2 * GMIN) >> 4) << 14));
        else if (NS > 2 && k >= 1)
            __builtin_amdgcn_s_waitcnt(0x0F70 | (GMIN & 15) | ((GMIN >> 4) << 14));
        else
            __builtin_amdgcn_s_waitcnt(0x0F70);
    };
    LaneOff woff[TN];
#pragma unroll
    for (int a = 0; a < TN; ++a)
        woff[a] = lane_off<FMT>(mat, min(row0 + 32 * a, mat.N - 1), h);
    // issue the loads of block blk (activations into buf, weights into w)
    auto issue = [&](int blk, uint8_t *buf, Raw<FMT> (&w)[TN]) {
        stage(buf, blk);
#pragma unroll
        for (int a = 0; a < TN; ++a)
            load_raw(w[a], mat, woff[a], blk);
        __builtin_amdgcn_sched_barrier(0);
    };

    // One 256-block: MFMAs on the activations in buf and the weights in
    // wcur, while the loads of block blk + NS - 1 (into nbuf, wnxt: the
    // buffers block blk - 1 used) are in flight.
    auto block = [&](int blk, const uint8_t *buf, uint8_t *nbuf, Raw<FMT> (&wcur)[TN],
                     Raw<FMT> (&wnxt)[TN]) {
        if (blk + NS - 1 < b1)
            issue(blk + NS - 1, nbuf, wnxt);
        const uint8_t *xa = buf + (wt * TM * 32 + r32) * RS + h * 16;
        floatx16 P[TN][TM];
#pragma unroll
        for (int a = 0; a < TN; ++a)
#pragma unroll
            for (int bb = 0; bb < TM; ++bb)
                zero16(P[a][bb]);

        // Software pipeline over the 16 k-steps: the A fragments (LDS) and B
        // fragments (decoded weights) of step s+1 are produced while the
        // MFMAs of step s run.
        Dec<FMT, WIDE> dec[TN];
        if constexpr (FMT != FMT_Q80) {
#pragma unroll
            for (int a = 0; a < TN; ++a)
                dec[a].init(wcur[a], h, g.nan_fb);
        }
        // Q8_0: the scales of this lane's blocks, 2h, 2h+1 (dlo) and 4+2h,
        // 5+2h (dhi) of the eight
        uint32_t dlo[TN], dhi[TN];
        if constexpr (FMT == FMT_Q80) {
#pragma unroll
            for (int a = 0; a < TN; ++a) {
                bad[a] |= q80_big_scale(wcur[a].d.x) | q80_big_scale(wcur[a].d.y) |
                          q80_big_scale(wcur[a].d.z) | q80_big_scale(wcur[a].d.w);
                dlo[a] = h ? wcur[a].d.y : wcur[a].d.x;
                dhi[a] = h ? wcur[a].d.w : wcur[a].d.z;
            }
        }
        auto afrag = [&](int s, half8_t (&A)[TM], half8_t (&AL)[TM]) {
#pragma unroll
            for (int bb = 0; bb < TM; ++bb) {
                A[bb] = lds_h8(xa + bb * 32 * RS + s * 32);
                if (SEP)
                    AL[bb] = lds_h8(xa + SROWS * RS + bb * 32 * RS + s * 32);
            }
        };
        auto bfrag = [&](int s, half8_t (&Bf)[TN], half8_t (&Bh)[TN]) {
#pragma unroll
            for (int a = 0; a < TN; ++a) {
                if constexpr (FMT == FMT_Q80) {
                    // k-step s = 2i + t: bytes 8t..8t+7 of load i, in Q8_0
                    // block 4(i&1) + 2h + i/4 of the eight, whose scale is
                    // splat to both halves
                    const int i = s >> 1;
                    const uint4 &qi = wcur[a].q[i];
                    const uint2 qq = (s & 1) ? make_uint2(qi.z, qi.w) : make_uint2(qi.x, qi.y);
                    const uint32_t dw = (i & 1) ? dhi[a] : dlo[a];
                    const uint32_t d2 = __builtin_amdgcn_perm(dw, dw, (i >> 2) ? 0x03020302u
                                                                               : 0x01000100u);
                    q80_split(qq, d2, Bf[a], Bh[a]);
                } else if constexpr (FMT == FMT_Q4K) {
                    Bf[a] = dec[a].frag(s);
                } else {
                    half2_t qv[4];
                    dec[a].quads(s, qv);
                    const int is = s >> 3, tp = s & 1;
                    const half2_t sl = dec[a].s2[is][tp], sh = dec[a].s2[is][tp + 2];
                    Bf[a] = h8(u32(qv[0] * sl), u32(qv[1] * sl), u32(qv[2] * sh), u32(qv[3] * sh));
                    if (WIDE) {
                        const half2_t wl = dec[a].s2h[is][tp], wh = dec[a].s2h[is][tp + 2];
                        Bh[a] = h8(u32(qv[0] * wl), u32(qv[1] * wl), u32(qv[2] * wh),
                                   u32(qv[3] * wh));
                    }
                }
            }
        };
        if constexpr (FMT == FMT_Q4K) {
            // min term: acc -= dmin * sum_g m_g Sx_g as two MFMAs on (Sx hi,
            // Sx lo) slots against (-dmin m) hi and lo (packed: the lo slot
            // rows of a token read the zero token, so only its hi slot row
            // carries the sums)
#pragma unroll
            for (int bb = 0; bb < TM; ++bb) {
                const half8_t am = lds_h8(buf + MOFF + (wt * TM * 32 + bb * 32 + r32) * MRS + h * 16);
#pragma unroll
                for (int a = 0; a < TN; ++a) {
                    acc[a][bb] = mfma32(am, h8(dec[a].mh[0], dec[a].mh[1], dec[a].mh[0], dec[a].mh[1]),
                                        acc[a][bb]);
                    acc[a][bb] = mfma32(am, h8(dec[a].ml[0], dec[a].ml[1], dec[a].ml[0], dec[a].ml[1]),
                                        acc[a][bb]);
                }
            }
        }
        half8_t A[2][TM], AL[2][TM], Bf[2][TN], Bh[2][TN];
        afrag(0, A[0], AL[0]);
        bfrag(0, Bf[0], Bh[0]);
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const int cu = s & 1;
            if (s + 1 < 16) {
                afrag(s + 1, A[cu ^ 1], AL[cu ^ 1]);
                bfrag(s + 1, Bf[cu ^ 1], Bh[cu ^ 1]);
            }
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
                for (int bb = 0; bb < TM; ++bb) {
                    // Q8_0's fragments carry d: its sums go straight into acc
                    floatx16 &T = FMT == FMT_Q80 ? acc[a][bb] : P[a][bb];
                    T = mfma32(A[cu][bb], Bf[cu][a], T);
                    if (SEP)
                        T = mfma32(AL[cu][bb], Bf[cu][a], T);
                    if (TWO) {
                        T = mfma32(A[cu][bb], Bh[cu][a], T);
                        if (SEP)
                            T = mfma32(AL[cu][bb], Bh[cu][a], T);
                    }
                }
#ifndef REALM_TILED_NO_SCHED
            // interleave: each MFMA of step s is followed by a share of the
            // LDS reads and the decode work of step s+1
            if (s + 1 < 16) {
                constexpr int NMF = TN * TM * (SEP ? 2 : 1) * (TWO ? 2 : 1);
                constexpr int NRD = TM * (SEP ? 2 : 1);
                constexpr int RPM = (NRD + NMF - 1) / NMF;
                constexpr int NVA = (FMT == FMT_Q4K ? 9 : 22) * TN;
                constexpr int VPM = (NVA + NMF - 1) / NMF;
#pragma unroll
                for (int m = 0; m < NMF; ++m) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, RPM, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
                }
            }
#endif
        }
        if constexpr (FMT != FMT_Q80) {
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
                for (int bb = 0; bb < TM; ++bb)
#pragma unroll
                    for (int v = 0; v < 16; ++v)
                        acc[a][bb][v] = __builtin_fmaf(dec[a].d, P[a][bb][v], acc[a][bb][v]);
        }
        // block blk + 1 has landed in LDS once this wave's loads for it are
        // done; then, after the barrier, every wave's are
        if (blk + 1 < b1) {
            __builtin_amdgcn_sched_barrier(0);
            const int later = min(b1 - 1, blk + NS - 1) - (blk + 1); // stages issued after it
            wait_stages(later);
        }
        lds_barrier();
    };

    // NS-stage pipeline: blocks b0 .. b0 + NS - 2 are issued up front; block
    // blk then uses buffer (blk - b0) % NS and weight set (blk - b0) % NS
    Raw<FMT> w[NS][TN];
#pragma unroll
    for (int u = 0; u < NS - 1; ++u)
        if (b0 + u < b1)
            issue(b0 + u, lbuf[u], w[u]);
    wait_stages(min(b1 - b0, NS - 1) - 1);
    lds_barrier();

    for (int base = b0; base < b1; base += NS) {
#pragma unroll
        for (int u = 0; u < NS; ++u) {
            if (base + u < b1)
                block(base + u, lbuf[u], lbuf[(u + NS - 1) % NS], w[u], w[(u + NS - 1) % NS]);
        }
    }

    // ---- epilogue: undo the token rescale.  All token scales are loaded
    // before the first store: a load issued after stores would wait for them
    // too (stores count in vmcnt).
    const int tw = m0 + wt * TM * TOK;
    float ts[TM][16];
#pragma unroll
    for (int bb = 0; bb < TM; ++bb)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            // slots 8 q4 + 4h + (0..3); tokens padded to GTOK have scales
            if (PACK) {
                const float2 t2 = *reinterpret_cast<const float2 *>(g.tscale + tw + 16 * bb + 4 * q4 + 2 * h);
                ts[bb][4 * q4] = ts[bb][4 * q4 + 1] = t2.x;
                ts[bb][4 * q4 + 2] = ts[bb][4 * q4 + 3] = t2.y;
            } else {
                const float4 t4 = *reinterpret_cast<const float4 *>(g.tscale + tw + 32 * bb + 8 * q4 + 4 * h);
                ts[bb][4 * q4] = t4.x;
                ts[bb][4 * q4 + 1] = t4.y;
                ts[bb][4 * q4 + 2] = t4.z;
                ts[bb][4 * q4 + 3] = t4.w;
            }
        }
    // the first 512 tokens' scales for the exact pass at the end, loaded
    // before the stores too (direct epilogue only)
    float tsv[8];
    if (!g.part) {
#pragma unroll
        for (int c = 0; c < 8; ++c)
            tsv[c] = g.tscale[min(64 * c + lane, g.M - 1)];
    }
    // this workgroup's sums: vals[bb][v / VS][a] for token slot(s) v of tile
    // bb (packed: slots v, v + 1 are one token's hi and lo), row tile a
    constexpr int VS = PACK ? 2 : 1, NV = 16 / VS;
    float vals[TM][NV][TN];
#pragma unroll
    for (int bb = 0; bb < TM; ++bb)
#pragma unroll
        for (int v = 0; v < 16; v += VS)
#pragma unroll
            for (int a = 0; a < TN; ++a)
                vals[bb][v / VS][a] = (PACK ? acc[a][bb][v] + acc[a][bb][v + 1] : acc[a][bb][v]) *
                                      ts[bb][v];
    // the position of value (bb, v, a) within the tile: token tl, row rl
    auto tloc = [&](int bb, int v) {
        const int slot = 8 * (v >> 2) + 4 * h + (v & 3);
        return wt * TM * TOK + (PACK ? 16 * bb + (slot >> 1) : 32 * bb + slot);
    };
    const int rl0 = wr * TN * 32 + r32; // + 32a
    if (g.part) {
        // this split's part of the tile (a K split, or one part when the
        // reduce also adds LoRA deltas); realm_gemm_tiled_reduce(_lora) adds
        // the parts in split order
        constexpr int TILE = GROWS * GTOK;
        float *pt = g.part + ((size_t)(rt * TT + tt) * KS + kc) * TILE;
#pragma unroll
        for (int bb = 0; bb < TM; ++bb)
#pragma unroll
            for (int v = 0; v < 16; v += VS)
#pragma unroll
                for (int a = 0; a < TN; ++a)
                    // a flagged Q8_0 row leaves NaN: the reduce recomputes it
                    pt[tloc(bb, v) * GROWS + rl0 + 32 * a] =
                        (FMT == FMT_Q80 && bad[a]) ? __builtin_nanf("") : vals[bb][v / VS][a];
        return;
    }
#pragma unroll
    for (int bb = 0; bb < TM; ++bb)
#pragma unroll
        for (int v = 0; v < 16; v += VS) {
            const int tok = m0 + tloc(bb, v);
            if (tok >= g.M)
                continue;
            // a token xprep flagged: the exact pass below writes it
            if (__builtin_expect(__builtin_isnan(ts[bb][v]), 0))
                continue;
#pragma unroll
            for (int a = 0; a < TN; ++a) {
                const int row = row0 + 32 * a;
                if (row >= mat.N)
                    continue;
                float out = vals[bb][v / VS][a];
                // a Q8_0 row with a scale d q in f16 cannot hold
                if (__builtin_expect(FMT == FMT_Q80 && bad[a], 0))
                    out = exact_dot<FMT>(mat.w0, mat.w1, mat.w2, row, g.K, g.KX,
                                         (const uint8_t *)g.x +
                                             (size_t)tok * g.K * (g.xbf16 ? 2 : 4),
                                         g.xbf16, g.nan_fb, 0, 1);
                yseg[(size_t)tok * mat.N + row] = out;
            }
        }
    // The flagged tokens' rows on the exact f32 path.  Every workgroup of
    // the row tile takes part, whichever token tile it holds (one flagged
    // token's rows would otherwise fall to the few workgroups of its own
    // tile while the rest of the chip idles): workgroup tt of TT takes rows
    // tt, tt + TT, ... of the tile for every flagged token, each wave every
    // (WR WT)-th of them, and each (row, token) is summed by one whole wave (k
    // split over its lanes; one lane walking all of K alone exposes every
    // weight load's latency, about 0.5 us per element).
    // The token scales are scanned 512 at a time, their loads issued
    // together (one memory round trip per 512 tokens; the first 512 were
    // loaded before the stores).
    for (int base = 0; base < g.M; base += 512) {
        if (base > 0) {
#pragma unroll
            for (int c = 0; c < 8; ++c)
                tsv[c] = g.tscale[min(base + 64 * c + lane, g.M - 1)];
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            unsigned long long fl = __ballot(base + 64 * c + lane < g.M && __builtin_isnan(tsv[c]));
            while (fl) {
                const int tok = base + 64 * c + (int)__builtin_ctzll(fl);
                fl &= fl - 1;
                const uint8_t *xt = (const uint8_t *)g.x + (size_t)tok * g.K * (g.xbf16 ? 2 : 4);
                for (int j = tt + TT * wave; j < GROWS; j += WR * WT * TT) {
                    const int row = rtl * GROWS + j;
                    if (row >= mat.N)
                        break;
                    const float out = exact_dot_wave<FMT>(mat.w0, mat.w1, mat.w2, row, g.K, g.KX,
                                                          xt, g.xbf16, g.nan_fb, lane);
                    if (lane == 0)
                        yseg[(size_t)tok * mat.N + row] = out;
                }
            }
        }
    }
}

// realm_gemm_<fmt>_t<WR><WT><TN><TM><p|s|b><NS>: NS pipeline stages; OCC
// waves per SIMD (2 caps a wave at 256 VGPRs so that two workgroups share a CU)
#define GEMM_TILED(FNAME, FMT, WIDE, WR, WT, TN, TM, MODE, MCODE, OCC, NS)                 \
    extern "C" __global__ __launch_bounds__(WR * WT * 64)                                  \
    __attribute__((amdgpu_waves_per_eu(OCC))) void                                          \
        realm_gemm_##FNAME##_t##WR##WT##TN##TM##MCODE##NS(GemmArgs g)                      \
    {                                                                                      \
        gemm_tiled<FMT, WR, WT, TN, TM, MODE, WIDE, NS>(g);                                \
    }
#define GEMM_TILED_SET(FNAME, FMT, WIDE)                                                   \
    GEMM_TILED(FNAME, FMT, WIDE, 4, 1, 1, 1, MODE_P, p, 2, 2)                              \
    GEMM_TILED(FNAME, FMT, WIDE, 4, 1, 1, 2, MODE_P, p, 2, 2)                              \
    GEMM_TILED(FNAME, FMT, WIDE, 4, 1, 1, 2, MODE_P, p, 1, 3)                              \
    GEMM_TILED(FNAME, FMT, WIDE, 8, 1, 1, 2, MODE_P, p, 1, 4)                              \
    GEMM_TILED(FNAME, FMT, WIDE, 4, 1, 1, 2, MODE_S, s, 1, 2)                              \
    GEMM_TILED(FNAME, FMT, WIDE, 4, 1, 1, 2, MODE_B, b, 2, 2)                              \
    GEMM_TILED(FNAME, FMT, WIDE, 4, 1, 1, 2, MODE_B, b, 1, 3)                              \
    GEMM_TILED(FNAME, FMT, WIDE, 4, 1, 1, 2, MODE_B, b, 1, 4)                              \
    GEMM_TILED(FNAME, FMT, WIDE, 8, 1, 1, 2, MODE_B, b, 1, 3)                              \
    GEMM_TILED(FNAME, FMT, WIDE, 8, 1, 1, 2, MODE_B, b, 1, 4)                              \
    GEMM_TILED(FNAME, FMT, WIDE, 4, 1, 1, 4, MODE_B, b, 1, 2)                              \
    GEMM_TILED(FNAME, FMT, WIDE, 8, 1, 1, 1, MODE_B, b, 1, 4)

// Q8_0 is compiled as a code object of its own (REALM_TILED_Q80), in
// parallel with the rest
#ifdef REALM_TILED_Q80
GEMM_TILED_SET(q80, FMT_Q80, false)
#else
GEMM_TILED_SET(q4k, FMT_Q4K, false)
GEMM_TILED_SET(q6k, FMT_Q6K, false)
GEMM_TILED_SET(q6kw, FMT_Q6K, true)

// y = the sum of a tiled launch's K-split parts, in split order (so results
// are deterministic).  Workgroup (tile, chunk): 256 of the tile's
// grows x gtok values; tile = row tile x token tiles + token tile, and the
// row tile's segment names the output matrix.
// Element e of tile `tile`: its segment (output matrix), row and token.
struct ReduceSite {
    int seg, N, row, tok, tl, rt, tt;
    float *y;
};
REALM_DEV ReduceSite reduce_site(const GemmArgs &g, int grows, int gtok, int tile, int e)
{
    ReduceSite r;
    const int TT = (g.M + gtok - 1) / gtok;
    r.rt = tile / TT;
    r.tt = tile - r.rt * TT;
    r.seg = (r.rt >= g.seg_tile[1]) + (r.rt >= g.seg_tile[2]) + (r.rt >= g.seg_tile[3]);
    auto pick = [&](auto a0, auto a1, auto a2, auto a3) {
        return r.seg == 0 ? a0 : r.seg == 1 ? a1 : r.seg == 2 ? a2 : a3;
    };
    r.N = pick(g.seg_n[0], g.seg_n[1], g.seg_n[2], g.seg_n[3]);
    r.y = pick(g.seg_y[0], g.seg_y[1], g.seg_y[2], g.seg_y[3]);
    const int rtl = r.rt - pick(g.seg_tile[0], g.seg_tile[1], g.seg_tile[2], g.seg_tile[3]);
    r.tl = e / grows;
    r.row = rtl * grows + (e - r.tl * grows);
    r.tok = r.tt * gtok + r.tl;
    return r;
}

// The base product of one element: the parts in split order, or the exact
// f32 dot product for a token xprep flagged and for a NaN sum (a Q8_0 row
// the tiled kernel flagged, or a NaN that the exact product reproduces).
// The sum of an element's ks parts (TILE apart) in split order, their loads
// issued 8 at a time (one memory round trip per 8 parts, not per part).
REALM_DEV float sum_parts(const float *p, int ks, int TILE)
{
    float sum = 0.f;
    for (int c0 = 0; c0 < ks; c0 += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (c0 + u < ks)
                v[u] = p[(size_t)(c0 + u) * TILE];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (c0 + u < ks)
                sum = c0 + u == 0 ? v[u] : sum + v[u];
    }
    return sum;
}

REALM_DEV float reduce_base(const GemmArgs &g, const ReduceSite &r, int tile, int e, int TILE)
{
    float sum = sum_parts(g.part + (size_t)tile * g.ksplit * TILE + e, g.ksplit, TILE);
    if (__builtin_expect(__builtin_isnan(g.tscale[r.tok]) || __builtin_isnan(sum), 0)) {
        auto pick = [&](auto a0, auto a1, auto a2, auto a3) {
            return r.seg == 0 ? a0 : r.seg == 1 ? a1 : r.seg == 2 ? a2 : a3;
        };
        const void *w0 = pick(g.seg_w0[0], g.seg_w0[1], g.seg_w0[2], g.seg_w0[3]);
        const void *w1 = pick(g.seg_w1[0], g.seg_w1[1], g.seg_w1[2], g.seg_w1[3]);
        const void *w2 = pick(g.seg_w2[0], g.seg_w2[1], g.seg_w2[2], g.seg_w2[3]);
        const uint8_t *x = (const uint8_t *)g.x + (size_t)r.tok * g.K * (g.xbf16 ? 2 : 4);
        // the reduce serves Q4_K, Q6_K and Q8_0 launches: the format from the layout
        sum = g.fmt == FMT_Q4K
                  ? exact_dot_ilp<FMT_Q4K>(w0, w1, w2, r.row, g.K, g.KX, x, g.xbf16, g.nan_fb, 0, 1)
              : g.fmt == FMT_Q6K
                  ? exact_dot_ilp<FMT_Q6K>(w0, w1, w2, r.row, g.K, g.KX, x, g.xbf16, g.nan_fb, 0, 1)
                  : exact_dot_ilp<FMT_Q80>(w0, w1, w2, r.row, g.K, g.KX, x, g.xbf16, g.nan_fb, 0, 1);
    }
    return sum;
}

extern "C" __global__ __launch_bounds__(256) void realm_gemm_tiled_reduce(GemmArgs g, int grows,
                                                                          int gtok)
{
    const int tile = blockIdx.x, e = blockIdx.y * 256 + threadIdx.x, TILE = grows * gtok;
    if (e >= TILE)
        return;
    const ReduceSite r = reduce_site(g, grows, gtok, tile, e);
    if (r.row >= r.N || r.tok >= g.M)
        return;
    r.y[(size_t)r.tok * r.N + r.row] = reduce_base(g, r, tile, e, TILE);
}

// The same, plus the multi-LoRA delta of the fused small-batch path:
//   y[t][n] = base + scale_a * sum_j u[t][j] B_a[n][j],  a = ids[t]
// (no delta for a = -1 or a slot past the projection's set), with u the sum
// of the fused shrink's parts.  A workgroup's 256 elements cover at most 3
// tokens (tiles have at least 128 rows); their u rows are summed into LDS,
// and each element takes its row of B_a in f32 FMAs.  Every global load (the
// base product's parts, the ids, the table entries, u and the first 256
// bytes of the B row) is issued before the one LDS barrier.  (An MFMA form,
// B staged once per tile and adapter, ran slower: its 125 KB of LDS left one
// 4-wave workgroup per CU and nothing to hide its dependent loads and
// barriers behind.)
extern "C" __global__ __launch_bounds__(256) void realm_gemm_tiled_reduce_lora(GemmArgs g,
                                                                               int grows, int gtok,
                                                                               LoraGroupArgs L)
{
    __shared__ float us[3][LORA_FUSED_RMAX];
    const int tile = blockIdx.x, e = blockIdx.y * 256 + threadIdx.x, TILE = grows * gtok;
    const ReduceSite r = reduce_site(g, grows, gtok, tile, e);
    const bool live = e < TILE && r.row < r.N && r.tok < g.M;
    auto lpick = [&](auto a0, auto a1, auto a2, auto a3) {
        return r.seg == 0 ? a0 : r.seg == 1 ? a1 : r.seg == 2 ? a2 : a3;
    };
    const LoraEntry *table = lpick(L.table[0], L.table[1], L.table[2], L.table[3]);
    const float *u = lpick(L.u[0], L.u[1], L.u[2], L.u[3]);
    const int rmax = lpick(L.rmax[0], L.rmax[1], L.rmax[2], L.rmax[3]);
    const int pstride = lpick(L.pstride[0], L.pstride[1], L.pstride[2], L.pstride[3]);
    const int nad = lpick(L.a_start[1], L.a_start[2], L.a_start[3], L.a_start[4]) -
                    lpick(L.a_start[0], L.a_start[1], L.a_start[2], L.a_start[3]);
    // the base product's parts
    float sum = 0.f;
    if (live) {
        sum = sum_parts(g.part + (size_t)tile * g.ksplit * TILE + e, g.ksplit, TILE);
    }
    // this element's adapter and its B row: up to 256 bytes in registers
    // when the row is 16-byte aligned (f16: ranks to 128, f32: to 64)
    const int a = live ? L.ids[r.tok] : -1;
    const bool has = a >= 0 && a < nad;
    LoraEntry en = {};
    uint4 braw[16];
    int nb = 0;
    if (has) {
        en = table[a];
        const size_t esz = en.dtype ? 2 : 4, rowbytes = (size_t)en.rank * esz;
        const uint8_t *bp = (const uint8_t *)en.b + (size_t)r.row * rowbytes;
        if ((rowbytes & 15) == 0 && ((uintptr_t)bp & 15) == 0)
            nb = (int)min(rowbytes >> 4, (size_t)16);
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (i < nb)
                braw[i] = ((gu4_t *)bp)[i];
    }
    // the u rows of the workgroup's tokens: tile-local tl0 .. tl0 + 2
    const int tl0 = (int)(blockIdx.y * 256) / grows;
#pragma unroll
    for (int q = 0; q < 3; ++q) {
        const int tq = r.tt * gtok + tl0 + q;
        const int aq = tl0 + q < gtok && tq < g.M ? L.ids[tq] : -1;
        if (aq < 0 || aq >= nad)
            continue;
        const int rank = table[aq].rank;
        for (int j = threadIdx.x; j < rank; j += 256) {
            const float *up = u + (size_t)tq * rmax + j;
            float s = up[0];
            for (int c = 1; c < L.nparts; ++c)
                s += up[(size_t)c * pstride];
            us[q][j] = s;
        }
    }
    lds_barrier();
    if (!live)
        return;
    if (__builtin_expect(__builtin_isnan(g.tscale[r.tok]) || __builtin_isnan(sum), 0))
        sum = reduce_base(g, r, tile, e, TILE); // flagged: the exact product
    if (has) {
        const float *uq = us[r.tl - tl0];
        float d = 0.f;
        if (en.dtype) {
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (i < nb) {
                    const half8_t h = __builtin_bit_cast(half8_t, braw[i]);
#pragma unroll
                    for (int q = 0; q < 8; ++q)
                        d = fmaf(uq[8 * i + q], (float)h[q], d);
                }
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (i < nb) {
                    const float4 f = __builtin_bit_cast(float4, braw[i]);
                    d = fmaf(uq[4 * i], f.x, d);
                    d = fmaf(uq[4 * i + 1], f.y, d);
                    d = fmaf(uq[4 * i + 2], f.z, d);
                    d = fmaf(uq[4 * i + 3], f.w, d);
                }
        }
        // the rest of the row (unaligned rows, f32 ranks past 64)
        int j = nb * (en.dtype ? 8 : 4);
        if (en.dtype) {
            gf16_t *bp = (gf16_t *)en.b + (size_t)r.row * en.rank;
            for (; j < en.rank; ++j)
                d = fmaf(uq[j], (float)bp[j], d);
        } else {
            gf32_t *bp = (gf32_t *)en.b + (size_t)r.row * en.rank;
            for (; j < en.rank; ++j)
                d = fmaf(uq[j], bp[j], d);
        }
        sum += en.scale * d;
    }
    r.y[(size_t)r.tok * r.N + r.row] = sum;
}
#endif // REALM_TILED_Q80

// Batched decode (M >= 2) and prefill: Y[t, n] = sum_k X[t,k] W[n,k] on MFMA
// (v_mfma_f32_16x16x32_f16, f32 accumulate) for resident Q4_K / Q6_K / Q8_0
// weights, plus the multi-LoRA shrink and the fused LoRA expand epilogue.
//
// Exactness: every MFMA operand is exact in f16.
//  * Activations: xprep rescales each token by an exact power of two 2^-e_t
//    (max |x| lands in [512, 1024)) and splits it into f16 hi + lo parts
//    (lo = 0 for bf16 input, which is exact in f16 after the rescale).  The
//    output is multiplied back by 2^e_t.
//  * Q4_K weights: sc*q with sc <= 63, q <= 15 (<= 945 < 2^11); per 256-block
//    the MFMA sum is scaled by d, and the min term dmin * sum_s m_s Sx_s runs
//    as one extra MFMA whose K slots hold (Sx hi, Sx lo) against (m, m).
//  * Q6_K weights: (q-32)*sc when every |sc| <= 63 (<= 2016 < 2^11); otherwise
//    sc = 16*sh + sl and two exact operands (q-32)*sl and (q-32)*16*sh.
//  * Q8_0 weights: q itself; each 32-block's MFMA sum is scaled by d.
//
// MFMA roles: A = activations (16 tokens x 32 k), B = weights (32 k x 16
// rows), D[token][row].  Lane l supplies A[l%16][kslot(l/16, e)] and
// B[kslot(l/16, e)][l%16]; the k slots of a lane group c = l/16 are chosen
// per format so that a lane reads contiguous weight bytes of its own row, and
// xprep writes activations in exactly that slot order.  D lane l holds rows
// 4(l/16)+v (tokens) of column l%16 (a row n), so each lane scales its own
// row's results with the block scale it decoded itself.
#include "mfma_common.h"
#include "kernel_args.h"

using namespace realm;

// ------------------------------------------------------------------ xprep
//
// One workgroup of 1024 threads per (padded) token.  Writes, for token t, in
// slot order ORD (mfma_common.h):
//   xh[t][p], xl[t][p]  f16 hi/lo of x[t][k(p)] * 2^-e_t, p in [0, KX)
//   xm                  Q4_K only, the 32-element sums Sx of x * 2^-e_t as
//                       f16 hi/lo, laid out as the min-term MFMA reads them:
//                       ORD 0: xm[t][b][c][8] = (Sxh(2c), Sxh(2c+1), Sxl(2c),
//                              Sxl(2c+1), 0, 0, 0, 0)
//                       ORD 1: xm[t][b][h][8] = (Sxh(4h..4h+3), Sxl(4h..4h+3))
//   tscale[t] = 2^e_t, or NaN when the token needs the exact path (exact.h:
//               a NaN / Inf element, or max |x| outside [EXACT_LO, EXACT_HI]);
//               its prepared activations are then zero
// Tokens t >= M get zeros.  Position group pg = p/8 (8 slots) is handled by
// thread pg % 1024: it loads the 8 x of its window once, takes part in the
// token's max, then converts them; the Q4_K sums come from the threads that
// share a sub-block (lanes of one 16-lane row).
#define XPREP_TH 1024
#define XPREP_R 4 // position-group rounds held in registers: KX <= 32768

template <int FMT, int ORD, int TH = XPREP_TH>
REALM_DEV void xprep(const void *__restrict__ x, int bf16, _Float16 *__restrict__ xh,
                     _Float16 *__restrict__ xl, _Float16 *__restrict__ xm,
                     float *__restrict__ tscale, int M, int K, int KX)
{
    __shared__ float red[TH / 64];
    const int t = blockIdx.x;
    const bool live = t < M;
    const size_t xrow = (size_t)t * K;
    const int ngroups = KX >> 3;
    constexpr int GAP = kgap<FMT, ORD>();
    float v[XPREP_R][8];
    float amax = 0.f;
#pragma unroll
    for (int r = 0; r < XPREP_R; ++r) {
        const int pg = r * TH + threadIdx.x;
        const int k0 = pg < ngroups ? kwin<FMT, ORD>(pg) : 0;
        // a window is 4 + 4 consecutive k (GAP apart): two vector loads when
        // both halves are inside the row (K % 4 == 0 keeps them aligned)
        const bool whole = live && pg < ngroups && k0 + GAP + 4 <= K && (K & 3) == 0 &&
                           ((uintptr_t)x & (bf16 ? 7u : 15u)) == 0;
        if (whole) {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const size_t i0 = xrow + k0 + GAP * hh;
                if (bf16) {
                    const uint2 b = *reinterpret_cast<const uint2 *>(
                        reinterpret_cast<const uint16_t *>(x) + i0);
                    v[r][4 * hh + 0] = __uint_as_float(b.x << 16);
                    v[r][4 * hh + 1] = __uint_as_float(b.x & 0xFFFF0000u);
                    v[r][4 * hh + 2] = __uint_as_float(b.y << 16);
                    v[r][4 * hh + 3] = __uint_as_float(b.y & 0xFFFF0000u);
                } else {
                    const float4 f = *reinterpret_cast<const float4 *>(
                        reinterpret_cast<const float *>(x) + i0);
                    v[r][4 * hh + 0] = f.x;
                    v[r][4 * hh + 1] = f.y;
                    v[r][4 * hh + 2] = f.z;
                    v[r][4 * hh + 3] = f.w;
                }
            }
        } else {
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                const int k = k0 + (w & 3) + GAP * (w >> 2);
                v[r][w] = (live && pg < ngroups && k < K) ? load_x(x, bf16, xrow + k) : 0.f;
            }
        }
        // a non-finite element counts as +Inf in the max (fmaxf would drop a NaN)
#pragma unroll
        for (int w = 0; w < 8; ++w)
            amax = fmaxf(amax, __builtin_isfinite(v[r][w]) ? fabsf(v[r][w]) : __builtin_inff());
    }
    // workgroup max: wave reduction (lane 63 ends with it), then LDS
    for (int off = 32; off > 0; off >>= 1)
        amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = 0.f;
#pragma unroll
    for (int w = 0; w < TH / 64; ++w)
        amax = fmaxf(amax, red[w]);
    const bool exact = exact_needed(amax, !__builtin_isfinite(amax));
    int e = 0;
    if (amax > 0.f && !exact) {
        int ex;
        frexpf(amax, &ex); // amax = m * 2^ex, m in [0.5, 1); |ex| <= 101 here
        e = ex - 10;
    }
    const float down = exact ? 0.f : ldexpf(1.f, -e);
    if (threadIdx.x == 0)
        tscale[t] = exact ? __builtin_nanf("") : ldexpf(1.f, e);

    const size_t orow = (size_t)t * KX;
    const int B = K >> 8;
#pragma unroll
    for (int r = 0; r < XPREP_R; ++r) {
        const int pg = r * TH + threadIdx.x;
        _Float16 hv[8], lv[8];
        float sum = 0.f, shi = 0.f; // of this thread's x * down: all 8 / the upper 4
#pragma unroll
        for (int s2 = 0; s2 < 8; ++s2) {
            const float val = exact ? 0.f : v[r][pi8(s2)] * down;
            const _Float16 h = (_Float16)val;
            hv[s2] = h;
            lv[s2] = (_Float16)(val - (float)h);
            if (ORD == 1 && s2 >= 4)
                shi += val;
            else
                sum += val;
        }
        if (pg < ngroups) {
            *reinterpret_cast<uint4 *>(xh + orow + 8 * pg) = __builtin_bit_cast(uint4, hv);
            if (xl)
                *reinterpret_cast<uint4 *>(xl + orow + 8 * pg) = __builtin_bit_cast(uint4, lv);
        }
        if (FMT == FMT_Q4K && ORD == 0) {
            // pg = 32b + 4i + c: the half group (b, c, h = i/4) is the four
            // threads pg, pg+4, pg+8, pg+12 of one 16-lane DPP row
            sum += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sum), 0x124, 0xF, 0xF, false)); // row_ror:4
            sum += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sum), 0x128, 0xF, 0xF, false)); // row_ror:8
            const int b = pg >> 5, i = (pg >> 2) & 7, c = pg & 3, h = i >> 2;
            if (pg < ngroups && b < B && (i & 3) == 0) {
                const _Float16 sh = (_Float16)sum;
                const _Float16 sl = (_Float16)(sum - (float)sh);
                _Float16 *dst = xm + ((size_t)t * B + b) * 32 + 8 * c;
                dst[h] = sh;
                dst[2 + h] = sl;
                if (h == 0)
                    *reinterpret_cast<uint2 *>(dst + 4) = make_uint2(0u, 0u);
            }
        }
        if (FMT == FMT_Q4K && ORD == 1) {
            // pg = 32b + 2s + h: sub-blocks 4h + 2(s/8) (lower 4 of each
            // window) and 4h + 2(s/8) + 1 (upper 4) gather the eight threads
            // with equal b, h, s/8, i.e. lanes that differ in bits 1..3
#pragma unroll
            for (int off = 2; off <= 8; off <<= 1) {
                sum += __shfl_xor(sum, off, 64);
                shi += __shfl_xor(shi, off, 64);
            }
            const int b = pg >> 5, q = (pg >> 4) & 1, h = pg & 1;
            if (pg < ngroups && b < B && (pg & 14) == 0) {
                _Float16 *dst = xm + (((size_t)t * B + b) * 2 + h) * 8;
                const _Float16 lh = (_Float16)sum, hh = (_Float16)shi;
                dst[2 * q] = lh;
                dst[2 * q + 4] = (_Float16)(sum - (float)lh);
                dst[2 * q + 1] = hh;
                dst[2 * q + 5] = (_Float16)(shi - (float)hh);
            }
        }
    }
}

#define DEF_XPREP(NAME, FMT)                                                               \
    extern "C" __global__ __launch_bounds__(XPREP_TH) void realm_xprep_##NAME(            \
        const void *x, int bf16, _Float16 *xh, _Float16 *xl, _Float16 *xm, float *tscale, \
        int M, int K, int KX)                                                              \
    {                                                                                      \
        xprep<FMT, 0>(x, bf16, xh, xl, xm, tscale, M, K, KX);                              \
    }                                                                                      \
    extern "C" __global__ __launch_bounds__(XPREP_TH) void realm_xprep_##NAME##_o1(       \
        const void *x, int bf16, _Float16 *xh, _Float16 *xl, _Float16 *xm, float *tscale, \
        int M, int K, int KX)                                                              \
    {                                                                                      \
        xprep<FMT, 1>(x, bf16, xh, xl, xm, tscale, M, K, KX);                              \
    }
DEF_XPREP(q4k, FMT_Q4K)
DEF_XPREP(q6k, FMT_Q6K)
DEF_XPREP(q80, FMT_Q80)

// The same with 256 threads per token for K <= 8192, 512 for K <= 16384
// (4 rounds of TH x 8 positions): every thread has work at 4096 (the
// 1024-thread form leaves half of them idle there), its loads issued
// together, and the token's max meets over fewer waves.
#define DEF_XPREP_TH(NAME, FMT, TH)                                                        \
    extern "C" __global__ __launch_bounds__(TH) void realm_xprep_##NAME##_t##TH(           \
        const void *x, int bf16, _Float16 *xh, _Float16 *xl, _Float16 *xm, float *tscale, \
        int M, int K, int KX)                                                              \
    {                                                                                      \
        xprep<FMT, 0, TH>(x, bf16, xh, xl, xm, tscale, M, K, KX);                          \
    }                                                                                      \
    extern "C" __global__ __launch_bounds__(TH) void realm_xprep_##NAME##_o1_t##TH(        \
        const void *x, int bf16, _Float16 *xh, _Float16 *xl, _Float16 *xm, float *tscale, \
        int M, int K, int KX)                                                              \
    {                                                                                      \
        xprep<FMT, 1, TH>(x, bf16, xh, xl, xm, tscale, M, K, KX);                          \
    }
DEF_XPREP_TH(q4k, FMT_Q4K, 256)
DEF_XPREP_TH(q6k, FMT_Q6K, 256)
DEF_XPREP_TH(q80, FMT_Q80, 256)
DEF_XPREP_TH(q4k, FMT_Q4K, 512)
DEF_XPREP_TH(q6k, FMT_Q6K, 512)
DEF_XPREP_TH(q80, FMT_Q80, 512)

// --------------------------------------------------------- LoRA adapter table

// Adapter factors are device allocations reached through pointers read from
// the adapter table: their loads go through the global address-space types
// of mfma_common.h (gf16_t, gf32_t, gu4_t, gu2_t, gf4_t).

REALM_DEV float lora_elem(const void *p, int dtype, size_t i)
{
    if (dtype)
        return (float)((gf16_t *)p)[i];
    return ((gf32_t *)p)[i];
}

// ------------------------------------------------------------- main kernel

// WAVES waves per workgroup: WAVES / KSPLIT along rows, KSPLIT along K.
// PACK (f32 activations only): the 16 MFMA token slots hold 8 tokens as
// (hi, lo) pairs, slot 2t + p = part p of token t, so one MFMA covers both
// parts and the epilogue adds the pair; otherwise a slot is one token and
// the lo part (LO) takes a second MFMA.
template <int FMT, int TN, int TM, int KSPLIT, bool LO, bool WIDE, int WAVES = 4,
          bool PACK = false>
REALM_DEV void gemm_body(const GemmArgs &g)
{
    constexpr int WN = WAVES / KSPLIT; // waves along rows
    constexpr bool SEP = LO && !PACK;  // separate MFMAs for the lo part
    constexpr int TOK = PACK ? 8 : 16; // tokens per 16-slot tile
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wn = wave / KSPLIT, wk = wave % KSPLIT;
    const int r16 = lane & 15, c = lane >> 4;
    const int n0 = blockIdx.x * (WN * 16 * TN) + wn * 16 * TN;
    const int t0 = blockIdx.y * (TOK * TM);
    const int K = g.K, KX = g.KX, N = g.N;

    floatx4 acc[TN][TM];
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
        for (int b = 0; b < TM; ++b)
            acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};

    // activation row pointers for this lane's slot in each token tile
    const _Float16 *xrow_h[TM];
    const _Float16 *xrow_l[TM];
#pragma unroll
    for (int b = 0; b < TM; ++b) {
        if (PACK) {
            size_t tok = (size_t)(t0 + TOK * b + (r16 >> 1));
            xrow_h[b] = (const _Float16 *)((r16 & 1) ? g.xl : g.xh) + tok * KX + 8 * c;
            xrow_l[b] = nullptr;
        } else {
            size_t tok = (size_t)(t0 + 16 * b + r16);
            xrow_h[b] = (const _Float16 *)g.xh + tok * KX + 8 * c;
            xrow_l[b] = LO ? (const _Float16 *)g.xl + tok * KX + 8 * c : nullptr;
        }
    }

    if (FMT == FMT_Q4K) {
        const int B = K >> 8;
        const uint8_t *hdr = (const uint8_t *)g.w0, *qs = (const uint8_t *)g.w1;
        for (int b = wk; b < B; b += KSPLIT) {
            uint32_t w[TN][8];
            float d[TN], dm[TN];
            half2_t sc2[TN][2], cc2[TN][2];
            uint32_t mfrag[TN];
#pragma unroll
            for (int a = 0; a < TN; ++a) {
                int row = n0 + 16 * a + r16;
                uint4 q0 = make_uint4(0, 0, 0, 0), q1 = q0, hd = q0;
                if (row < N) {
                    const size_t U = (size_t)(K >> 6);
                    const uint8_t *qp = qs + (size_t)row * (U * 32) + (4 * b + c) * 16;
                    q0 = ldg16(qp);          // plane 0
                    q1 = ldg16(qp + U * 16); // plane 1
                    hd = ldg16(hdr + ((size_t)row * B + b) * 16);
                }
                // the device layout stores high nibbles XOR 8: undo it here
                w[a][0] = q0.x ^ 0x80808080u; w[a][1] = q0.y ^ 0x80808080u;
                w[a][2] = q0.z ^ 0x80808080u; w[a][3] = q0.w ^ 0x80808080u;
                w[a][4] = q1.x ^ 0x80808080u; w[a][5] = q1.y ^ 0x80808080u;
                w[a][6] = q1.z ^ 0x80808080u; w[a][7] = q1.w ^ 0x80808080u;
                d[a] = fix_scale(f16_bits_to_f32(hd.x), 0.00000006f, g.nan_fb);
                dm[a] = fix_scale(f16_bits_to_f32(hd.x >> 16), 0.00000024f, g.nan_fb);
                // scale/min pair of sub-blocks 2c (low nibbles) and 2c+1 (high)
                const uint32_t pr = q4k_dev_pair(hd.y, hd.z, hd.w, c);
                const uint32_t sl = pr & 63u, ml = (pr >> 6) & 63u;
                const uint32_t shh = (pr >> 12) & 63u, mh = (pr >> 18) & 63u;
                sc2[a][0] = splat2((float)sl);
                cc2[a][0] = splat2(-1024.f * (float)sl);
                sc2[a][1] = splat2((float)shh);
                cc2[a][1] = splat2(-1024.f * (float)shh);
                half2_t mm = {(_Float16)(float)ml, (_Float16)(float)mh};
                mfrag[a] = u32(mm);
            }
            floatx4 P[TN][TM];
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
                for (int bb = 0; bb < TM; ++bb)
                    P[a][bb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                half8_t ah[TM], al[TM];
#pragma unroll
                for (int bb = 0; bb < TM; ++bb) {
                    ah[bb] = ld_h8(xrow_h[bb] + 256 * b + 32 * i);
                    if (SEP)
                        al[bb] = ld_h8(xrow_l[bb] + 256 * b + 32 * i);
                }
#pragma unroll
                for (int a = 0; a < TN; ++a) {
                    const int ch = i & 3, hi = i >> 2, shf = 4 * hi;
                    uint32_t wa = w[a][2 * ch], wb = w[a][2 * ch + 1];
                    uint32_t p0 = ((wa >> shf) & 0x000F000Fu) | 0x64006400u;
                    uint32_t p1 = ((wa >> (shf + 8)) & 0x000F000Fu) | 0x64006400u;
                    uint32_t p2 = ((wb >> shf) & 0x000F000Fu) | 0x64006400u;
                    uint32_t p3 = ((wb >> (shf + 8)) & 0x000F000Fu) | 0x64006400u;
                    half2_t s2 = sc2[a][hi], k2 = cc2[a][hi];
                    half8_t bf = h8(u32(__builtin_elementwise_fma(h2(p0), s2, k2)),
                                    u32(__builtin_elementwise_fma(h2(p1), s2, k2)),
                                    u32(__builtin_elementwise_fma(h2(p2), s2, k2)),
                                    u32(__builtin_elementwise_fma(h2(p3), s2, k2)));
#pragma unroll
                    for (int bb = 0; bb < TM; ++bb) {
                        P[a][bb] = mfma(ah[bb], bf, P[a][bb]);
                        if (SEP)
                            P[a][bb] = mfma(al[bb], bf, P[a][bb]);
                    }
                }
            }
            // min term: one MFMA on (Sx hi, Sx lo) x (m, m) slots
#pragma unroll
            for (int bb = 0; bb < TM; ++bb) {
                // packed: the hi slot of a token carries its whole min term
                size_t tok = PACK ? (size_t)(t0 + TOK * bb + (r16 >> 1)) : (size_t)(t0 + 16 * bb + r16);
                half8_t am = ld_h8((const _Float16 *)g.xm + (tok * B + b) * 32 + 8 * c);
                if (PACK && (r16 & 1))
                    am = half8_t{};
#pragma unroll
                for (int a = 0; a < TN; ++a) {
                    half8_t bm = h8(mfrag[a], mfrag[a], 0u, 0u);
                    floatx4 Q = mfma(am, bm, floatx4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        acc[a][bb][v] += d[a] * P[a][bb][v] - dm[a] * Q[v];
                }
            }
        }
    } else if (FMT == FMT_Q6K) {
        const int B = K >> 8;
        const uint8_t *dq = (const uint8_t *)g.w0;
        const int8_t *scq = (const int8_t *)g.w1;
        const uint8_t *qq = (const uint8_t *)g.w2;
        for (int b = wk; b < B; b += KSPLIT) {
            uint32_t qa[TN][4], qb[TN][4], qh[TN][4];
            float d[TN];
            half2_t s2[TN][4], s2h[TN][4];
#pragma unroll
            for (int a = 0; a < TN; ++a) {
                int row = n0 + 16 * a + r16;
                uint4 A = make_uint4(0, 0, 0, 0), Bq = A, H = A;
                uint32_t scw = 0, dbits = 0;
                if (row < N) {
                    size_t blk = (size_t)row * B + b, U = 4 * (size_t)B;
                    const uint8_t *qp = qq + (size_t)row * (U * 48) + (4 * b + c) * 16;
                    A = ldg16(qp);
                    Bq = ldg16(qp + U * 16);
                    H = ldg16(qp + U * 32);
                    scw = ldg4(scq + blk * 16 + 4 * c);
                    dbits = *reinterpret_cast<const uint16_t *>(dq + blk * 2);
                }
                qa[a][0] = A.x; qa[a][1] = A.y; qa[a][2] = A.z; qa[a][3] = A.w;
                qb[a][0] = Bq.x; qb[a][1] = Bq.y; qb[a][2] = Bq.z; qb[a][3] = Bq.w;
                qh[a][0] = H.x; qh[a][1] = H.y; qh[a][2] = H.z; qh[a][3] = H.w;
                d[a] = fix_scale(f16_bits_to_f32(dbits), 0.00000006f, g.nan_fb);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    int sc = (int)(int8_t)(scw >> (8 * t));
                    if (WIDE) {
                        s2[a][t] = splat2((float)(sc & 15));
                        s2h[a][t] = splat2(16.f * (float)(sc >> 4));
                    } else {
                        s2[a][t] = splat2((float)sc);
                    }
                }
            }
            floatx4 P[TN][TM];
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
                for (int bb = 0; bb < TM; ++bb)
                    P[a][bb] = floatx4{0.f, 0.f, 0.f, 0.f};
            const half2_t off2 = splat2(-1056.f);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int t = i >> 1, jh = i & 1;
                half8_t ah[TM], al[TM];
#pragma unroll
                for (int bb = 0; bb < TM; ++bb) {
                    ah[bb] = ld_h8(xrow_h[bb] + 256 * b + 32 * i);
                    if (SEP)
                        al[bb] = ld_h8(xrow_l[bb] + 256 * b + 32 * i);
                }
#pragma unroll
                for (int a = 0; a < TN; ++a) {
                    uint32_t v[2];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        uint32_t src = (t & 1) ? qb[a][2 * jh + h] : qa[a][2 * jh + h];
                        uint32_t lo4 = (src >> ((t & 2) ? 4 : 0)) & 0x0F0F0F0Fu;
                        uint32_t hi2 = ((qh[a][2 * jh + h] >> (2 * t)) & 0x03030303u) << 4;
                        v[h] = lo4 | hi2;
                    }
                    half2_t q0 = h2((v[0] & 0x00FF00FFu) | 0x64006400u) + off2;
                    half2_t q1 = h2(((v[0] >> 8) & 0x00FF00FFu) | 0x64006400u) + off2;
                    half2_t q2 = h2((v[1] & 0x00FF00FFu) | 0x64006400u) + off2;
                    half2_t q3 = h2(((v[1] >> 8) & 0x00FF00FFu) | 0x64006400u) + off2;
                    half2_t s = s2[a][t];
                    half8_t bf = h8(u32(q0 * s), u32(q1 * s), u32(q2 * s), u32(q3 * s));
                    half8_t bh;
                    if (WIDE) {
                        half2_t sh = s2h[a][t];
                        bh = h8(u32(q0 * sh), u32(q1 * sh), u32(q2 * sh), u32(q3 * sh));
                    }
#pragma unroll
                    for (int bb = 0; bb < TM; ++bb) {
                        P[a][bb] = mfma(ah[bb], bf, P[a][bb]);
                        if (SEP)
                            P[a][bb] = mfma(al[bb], bf, P[a][bb]);
                        if (WIDE) {
                            P[a][bb] = mfma(ah[bb], bh, P[a][bb]);
                            if (SEP)
                                P[a][bb] = mfma(al[bb], bh, P[a][bb]);
                        }
                    }
                }
            }
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
                for (int bb = 0; bb < TM; ++bb)
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        acc[a][bb][v] += d[a] * P[a][bb][v];
        }
    } else { // Q8_0
        const int B32 = KX >> 5;
        const uint8_t *dq = (const uint8_t *)g.w0;
        const int8_t *qq = (const int8_t *)g.w1;
        const half2_t off2 = splat2(-1152.f);
        for (int kb = wk; kb < B32; kb += KSPLIT) {
            half8_t ah[TM], al[TM];
#pragma unroll
            for (int bb = 0; bb < TM; ++bb) {
                ah[bb] = ld_h8(xrow_h[bb] + 32 * kb);
                if (SEP)
                    al[bb] = ld_h8(xrow_l[bb] + 32 * kb);
            }
#pragma unroll
            for (int a = 0; a < TN; ++a) {
                int row = n0 + 16 * a + r16;
                uint2 q = make_uint2(0, 0);
                uint32_t dbits = 0;
                if (row < N) {
                    // bytes 32kb + 8c .. +7 of the row: unit kb/2, byte 32(kb&1)
                    // + 8c -> plane 2(kb&1) + c/2, offset 8(c&1)
                    const size_t U = (size_t)(KX >> 6);
                    q = ldg8(qq + (size_t)row * KX + (2 * (kb & 1) + (c >> 1)) * (U * 16) +
                             (kb >> 1) * 16 + 8 * (c & 1));
                    dbits = *reinterpret_cast<const uint16_t *>(dq + ((size_t)row * B32 + kb) * 2);
                }
                float d = f16_bits_to_f32(dbits);
                uint32_t ua = q.x ^ 0x80808080u, ub = q.y ^ 0x80808080u;
                half2_t q0 = h2((ua & 0x00FF00FFu) | 0x64006400u) + off2;
                half2_t q1 = h2(((ua >> 8) & 0x00FF00FFu) | 0x64006400u) + off2;
                half2_t q2 = h2((ub & 0x00FF00FFu) | 0x64006400u) + off2;
                half2_t q3 = h2(((ub >> 8) & 0x00FF00FFu) | 0x64006400u) + off2;
                half8_t bf = h8(u32(q0), u32(q1), u32(q2), u32(q3));
#pragma unroll
                for (int bb = 0; bb < TM; ++bb) {
                    floatx4 P = mfma(ah[bb], bf, floatx4{0.f, 0.f, 0.f, 0.f});
                    if (SEP)
                        P = mfma(al[bb], bf, P);
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        acc[a][bb][v] += d * P[v];
                }
            }
        }
    }

    // ---- reduce the KSPLIT partial sums through LDS
    if (KSPLIT > 1) {
        __shared__ float red[WAVES][TN * TM * 4][64];
        if (wk != 0)
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
                for (int bb = 0; bb < TM; ++bb)
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        red[wave][(a * TM + bb) * 4 + v][lane] = acc[a][bb][v];
        __syncthreads();
        if (wk != 0)
            return;
#pragma unroll
        for (int s = 1; s < KSPLIT; ++s)
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
                for (int bb = 0; bb < TM; ++bb)
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        acc[a][bb][v] += red[wave + s][(a * TM + bb) * 4 + v][lane];
    }

    // ---- epilogue: undo the token rescale and store.  The token scales are
    // loaded before the first store: a load issued after stores would wait
    // for them too (stores count in vmcnt).
    float ts[TM][4];
#pragma unroll
    for (int bb = 0; bb < TM; ++bb)
#pragma unroll
        for (int v = 0; v < 4; v += (PACK ? 2 : 1)) {
            const int tok = PACK ? t0 + TOK * bb + 2 * c + (v >> 1) : t0 + 16 * bb + 4 * c + v;
            ts[bb][v] = g.tscale[tok]; // tokens are padded to the tile: every one has a scale
        }
#pragma unroll
    for (int bb = 0; bb < TM; ++bb)
#pragma unroll
        for (int v = 0; v < 4; v += (PACK ? 2 : 1)) {
            // packed: D rows 4c+v, 4c+v+1 are the (hi, lo) parts of one token
            int tok = PACK ? t0 + TOK * bb + 2 * c + (v >> 1) : t0 + 16 * bb + 4 * c + v;
            if (tok >= g.M)
                continue;
#pragma unroll
            for (int a = 0; a < TN; ++a) {
                int row = n0 + 16 * a + r16;
                if (row >= N)
                    continue;
                float sum = PACK ? acc[a][bb][v] + acc[a][bb][v + 1] : acc[a][bb][v];
                float out = sum * ts[bb][v];
                if (__builtin_expect(__builtin_isnan(ts[bb][v]), 0)) // flagged by xprep
                    out = exact_dot<FMT>(g.w0, g.w1, g.w2, row, g.K, g.KX,
                                         (const uint8_t *)g.x +
                                             (size_t)tok * g.K * (g.xbf16 ? 2 : 4),
                                         g.xbf16, g.nan_fb, 0, 1);
                g.y[(size_t)tok * N + row] = out;
            }
        }
}

#define GEMM_KERNEL(NAME, FMT, TN, TM, KS, LO, WIDE)                                      \
    extern "C" __global__ __launch_bounds__(256) void realm_gemm_##NAME(GemmArgs g)       \
    {                                                                                     \
        gemm_body<FMT, TN, TM, KS, LO, WIDE>(g);                                          \
    }
// Small batches: one 16-row tile per workgroup with K split over all of its
// 16/TM waves (more loads in flight per CU; the register budget of TM token
// tiles bounds the wave count); f32 activations pack (hi, lo) slots.
#define GEMM_KERNEL_S(NAME, FMT, TM, LO, WIDE)                                            \
    extern "C" __global__ __launch_bounds__(1024 / (TM)) void realm_gemm_##NAME(          \
        GemmArgs g)                                                                       \
    {                                                                                     \
        gemm_body<FMT, 1, TM, 16 / (TM), LO, WIDE, 16 / (TM), LO>(g);                      \
    }

// Instantiation set: (TN, TM, KSPLIT) tiles for decode (KSPLIT 4, TN 1) and
// prefill (KSPLIT 1, TN 2); LO = f32 activations; Q6_K narrow/wide scales.
#define GEMM_SMALL(FNAME, FMT, WIDE)                                                      \
    GEMM_KERNEL_S(FNAME##_s1_f32, FMT, 1, true, WIDE)                                     \
    GEMM_KERNEL_S(FNAME##_s2_f32, FMT, 2, true, WIDE)                                     \
    GEMM_KERNEL_S(FNAME##_s4_f32, FMT, 4, true, WIDE)                                     \
    GEMM_KERNEL_S(FNAME##_s1_bf16, FMT, 1, false, WIDE)                                   \
    GEMM_KERNEL_S(FNAME##_s2_bf16, FMT, 2, false, WIDE)
#define GEMM_TILES(FNAME, FMT, WIDE)                                                      \
    GEMM_SMALL(FNAME, FMT, WIDE)                                                          \
    GEMM_KERNEL(FNAME##_d1_f32, FMT, 1, 1, 4, true, WIDE)                                 \
    GEMM_KERNEL(FNAME##_d2_f32, FMT, 1, 2, 4, true, WIDE)                                 \
    GEMM_KERNEL(FNAME##_d4_f32, FMT, 1, 4, 4, true, WIDE)                                 \
    GEMM_KERNEL(FNAME##_p4_f32, FMT, 2, 4, 1, true, WIDE)                                 \
    GEMM_KERNEL(FNAME##_d1_bf16, FMT, 1, 1, 4, false, WIDE)                               \
    GEMM_KERNEL(FNAME##_d4_bf16, FMT, 1, 4, 4, false, WIDE)                               \
    GEMM_KERNEL(FNAME##_p4_bf16, FMT, 2, 4, 1, false, WIDE)

GEMM_TILES(q4k, FMT_Q4K, false)
GEMM_TILES(q6k, FMT_Q6K, false)
GEMM_TILES(q6kw, FMT_Q6K, true)
GEMM_TILES(q80, FMT_Q80, false)

// ------------------------------------------------------------ LoRA shrink
//
// The tokens of adapter a, in token order, compacted into LDS by the whole
// workgroup (a ballot per wave and a prefix over the waves); at most 1024
// (the host rejects larger batches).
REALM_DEV void adapter_tokens(const int *__restrict__ ids, int M, int a, int *toks, int *count,
                              int *wsum)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nwaves = blockDim.x >> 6;
    int base_pos = 0;
    for (int base = 0; base < M; base += blockDim.x) {
        const int t = base + threadIdx.x;
        const bool hit = t < M && ids[t] == a;
        const unsigned long long m = __ballot(hit);
        if (lane == 0)
            wsum[wave] = __popcll(m);
        __syncthreads();
        int before = base_pos;
        for (int w = 0; w < wave; ++w)
            before += wsum[w];
        int total = 0;
        for (int w = 0; w < nwaves; ++w)
            total += wsum[w];
        if (hit) {
            const int pos = before + __popcll(m & ((1ull << lane) - 1ull));
            if (pos < 1024)
                toks[pos] = t;
        }
        base_pos += total;
        __syncthreads();
    }
    if (threadIdx.x == 0)
        *count = base_pos < 1024 ? base_pos : 1024;
    __syncthreads();
}

// Shrink, u = A_a x, in parts over K: for the tokens t whose adapter is a and
// j < rank_a,
//   part[kc][t][j] = sum over positions [512 kc, 512 kc + 512) of
//                    A_a[j][k(p)] x[t][k(p)]
// (the expand adds the parts in kc order).  Grid (adapter, 16-row chunk of
// A, 512-position chunk kc), so that a launch spreads over many CUs; the 4
// waves take the adapter's tokens 16 at a time and the chunk's A fragments
// stay in registers across them.  Activations are the xprep fragments of the
// base matmul (slot order ORD, that of the base kernel); an adapter row's k
// window of a slot group is one or two vector loads, permuted to the slot
// order and split into f16 hi/lo (exact for f16 adapters, whose lo part is
// zero and skipped).
#define SHRINK_KC 512
#define SHRINK_NS (SHRINK_KC / 32)
template <int FMT, bool LO, int ORD, bool F16A>
REALM_DEV void shrink_body(const _Float16 *__restrict__ xh, const _Float16 *__restrict__ xl,
                           const float *__restrict__ tscale, const void *__restrict__ x,
                           int xbf16, const LoraEntry &e, const int *toks, int count,
                           float *__restrict__ part, int K, int KX, int rmax, int pstride)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r16 = lane & 15, c = lane >> 4;
    const int jc = blockIdx.y * 16, kc = blockIdx.z;
    const int j = jc + r16;
    // every load below reads valid memory: rows past the rank read the last
    // row and token slots past the adapter's tokens read its first token;
    // they only feed D rows / columns that are never stored.  Steps past the
    // chunk (s >= ns) are zeroed.
    const int jr = min(j, e.rank - 1);
    const int s0 = kc * SHRINK_NS;
    const int ns = min(SHRINK_NS, KX / 32 - s0); // 32-position steps in this chunk
    constexpr int GAP = kgap<FMT, ORD>();        // second 4 of a window at k0 + GAP
    half8_t bh[SHRINK_NS], bl[SHRINK_NS];
#pragma unroll
    for (int s = 0; s < SHRINK_NS; ++s) {
        // a window at or past K (Q8_0 rows padded to KX) reads nothing: the
        // adapter row has K entries
        const int kw = kwin<FMT, ORD>(4 * (s0 + min(s, ns - 1)) + c);
        const bool inrow = kw < K;
        const int k0 = inrow ? kw : 0;
        float v[8];
        if (F16A) {
            gf16_t *src = (gf16_t *)e.a + (size_t)jr * K + k0;
            const uint2 r0 = *(gu2_t *)src, r1 = *(gu2_t *)(src + GAP);
            const half8_t hv = __builtin_bit_cast(half8_t, make_uint4(r0.x, r0.y, r1.x, r1.y));
#pragma unroll
            for (int q = 0; q < 8; ++q)
                v[q] = (float)hv[q];
        } else {
            gf32_t *src = (gf32_t *)e.a + (size_t)jr * K + k0;
            const float4 f0 = *(gf4_t *)src;
            const float4 f1 = *(gf4_t *)(src + GAP);
            v[0] = f0.x; v[1] = f0.y; v[2] = f0.z; v[3] = f0.w;
            v[4] = f1.x; v[5] = f1.y; v[6] = f1.z; v[7] = f1.w;
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float vv = s < ns && inrow ? v[pi8(q)] : 0.f;
            const _Float16 hq = (_Float16)vv;
            bh[s][q] = hq;
            bl[s][q] = (_Float16)(vv - (float)hq);
        }
    }
    float *pk = part + (size_t)kc * pstride;
    for (int tc = 16 * wave; tc < count; tc += 64) {
        const int ti = tc + r16;
        const int tok = toks[ti < count ? ti : 0];
        floatx4 P = {0.f, 0.f, 0.f, 0.f};
        // the chunk's steps in two halves: each half's activation loads are
        // all in flight before its first MFMA (left alone, the scheduler
        // interleaves them with the MFMAs, one memory round trip per two
        // steps); halves keep the registers at two waves per SIMD
        constexpr int HS = SHRINK_NS / 2;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            half8_t ah[HS], al[HS];
#pragma unroll
            for (int i = 0; i < HS; ++i) {
                const int sc = s0 + min(hf * HS + i, ns - 1);
                ah[i] = ld_h8(xh + (size_t)tok * KX + 32 * sc + 8 * c);
                if (LO)
                    al[i] = ld_h8(xl + (size_t)tok * KX + 32 * sc + 8 * c);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < HS; ++i) {
                const int s = hf * HS + i;
                P = mfma(ah[i], bh[s], P);
                if (!F16A)
                    P = mfma(ah[i], bl[s], P);
                if (LO)
                    P = mfma(al[i], bh[s], P);
            }
        }
        float ts[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int tj = tc + 4 * c + v;
            ts[v] = tscale[toks[tj < count ? tj : 0]];
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            // D[token slot 4c+v][adapter row r16]; a token on the exact path
            // (NaN scale, prepared activations zero) holds 0 in parts past
            // the first, and the first is written below
            const int tj = tc + 4 * c + v;
            const bool ex = __builtin_isnan(ts[v]);
            if (tj < count && j < e.rank && !(ex && kc == 0))
                pk[(size_t)toks[tj] * rmax + j] = ex ? 0.f : P[v] * ts[v];
        }
        // Tokens on the exact path (a NaN / Inf element, or max |x| outside
        // the range the f16 split covers) get u in plain f32 from the
        // caller's activations: whole rows, in the first part, the wave's 64
        // lanes striding K for each of the chunk's 16 adapter rows.
        unsigned long long exm =
            __ballot(ti < count && __builtin_isnan(tscale[tok])) & 0xFFFFull; // slots r16
        if (kc != 0)
            exm = 0;
        while (exm) { // uniform
            const int te = toks[tc + __builtin_ctzll(exm)];
            exm &= exm - 1;
            for (int rr = 0; rr < 16 && jc + rr < e.rank; ++rr) {
                float acc = 0.f;
                for (int k = lane; k < K; k += 64)
                    acc = fmaf(lora_elem(e.a, e.dtype, (size_t)(jc + rr) * K + k),
                               load_x(x, xbf16, (size_t)te * K + k), acc);
                for (int off = 32; off > 0; off >>= 1)
                    acc += __shfl_xor(acc, off, 64);
                if (lane == 0)
                    pk[(size_t)te * rmax + jc + rr] = acc;
            }
        }
    }
}

// Projection p of a grouped LoRA launch that concatenated adapter slot ga
// falls in, and p's entry of a per-projection field (selects, not an
// indexed load: an indexed kernel-argument array would go to scratch).
REALM_DEV int lora_proj(const LoraGroupArgs &g, int ga)
{
    return (ga >= g.a_start[1] ? 1 : 0) + (ga >= g.a_start[2] ? 1 : 0) +
           (ga >= g.a_start[3] ? 1 : 0);
}
template <class T, int N>
REALM_DEV T lora_pick(const T (&v)[N], int p)
{
    static_assert(N >= REALM_GEMM_MAX_SEGS, "one entry per projection");
    return p == 0 ? v[0] : (p == 1 ? v[1] : (p == 2 ? v[2] : v[3]));
}

template <int FMT, bool LO, int ORD>
REALM_DEV void lora_shrink(const LoraGroupArgs &g)
{
    __shared__ int toks[1024];
    __shared__ int count;
    __shared__ int wsum[4];
    const int p = lora_proj(g, blockIdx.x);
    const int a = blockIdx.x - lora_pick(g.a_start, p);
    const auto *xh = (const _Float16 *)g.xh, *xl = (const _Float16 *)g.xl;
    float *part = lora_pick(g.u, p);
    const int rmax = lora_pick(g.rmax, p), pstride = lora_pick(g.pstride, p);
    adapter_tokens(g.ids, g.M, a, toks, &count, wsum);
    const LoraEntry e = lora_pick(g.table, p)[a];
    if ((int)blockIdx.y * 16 >= e.rank || count == 0)
        return;
    if (e.dtype)
        shrink_body<FMT, LO, ORD, true>(xh, xl, g.tscale, g.x, g.xbf16, e, toks, count, part,
                                        g.K, g.KX, rmax, pstride);
    else
        shrink_body<FMT, LO, ORD, false>(xh, xl, g.tscale, g.x, g.xbf16, e, toks, count, part,
                                         g.K, g.KX, rmax, pstride);
}

// ------------------------------------------------- fused LoRA shrink
//
// Small batches (the tiled base product with its K-split reduce): the shrink
// u = A_a x runs in workgroups of the xprep launch past its token rows, so a
// multi-LoRA call has the launches of a base call.  It cannot use xprep's
// fragments (written by the same launch) and reads the caller's activations
// instead (f32: the multi-LoRA calls take f32 activations), in natural k
// order, split into bf16 terms: x = b1 + b2 + b3 exactly (8 + 8 + 8
// significand bits), A = a1 + a2
// exactly for f16 factors (11 bits), a1 + a2 + a3 for f32 ones.  bf16 has
// f32's exponent range, so no scale is needed at any magnitude; the MFMAs
// take the terms of the products down to 2^-16 of the leading one (the ones
// left out are below 2^-24 of it) and accumulate in f32.  NaN and Inf
// elements give a NaN u, as f32 arithmetic would on the same row.
//
// Workgroup (projection, adapter slot, 16-row chunk of A, K part of
// LORA_FUSED_KP positions); its 16 waves share the part's 32-position steps
// (wave w: steps w, w + 16, ...) for each 16 of the adapter's tokens and sum
// through LDS:  u[part][t][j] for the adapter's tokens t and rows j < rank.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

REALM_DEV floatx4 mfma_bf(bf16x8_t a, bf16x8_t b, floatx4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// v = t1 + t2 (+ t3) in bf16, each term the rounding of what the ones
// before it leave (a non-finite leading term leaves 0)
template <int NT>
REALM_DEV void bf_split(const float (&v)[8], bf16x8_t &t1, bf16x8_t &t2, bf16x8_t &t3)
{
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const __bf16 h1 = (__bf16)v[i];
        const float r1 = __builtin_isfinite((float)h1) ? v[i] - (float)h1 : 0.f;
        t1[i] = h1;
        if (NT >= 2) {
            const __bf16 h2 = (__bf16)r1;
            t2[i] = h2;
            if (NT >= 3)
                t3[i] = (__bf16)(r1 - (float)h2);
        }
    }
}

#define FS_SW (LORA_FUSED_KP / 32 / 16) // steps per wave and part

// One workgroup's chunk: adapter slot a (entry e), rows jc .. jc + 15, K
// positions k0 .. k1 - 1.  idv is ids[threadIdx.x] (-1 past the batch).
template <bool F16A>
REALM_DEV void shrink_fused_body(const float *__restrict__ x, int K, const LoraEntry &e, int a,
                                 int idv, float *__restrict__ pk, int jc, int k0, int k1,
                                 int rmax, int *toks, int *wsum, float (*red)[256])
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r16 = lane & 15, c = lane >> 4;
    const int jr = min(jc + r16, e.rank - 1); // rows past the rank are never stored
    // A fragments: their loads go out first (they do not depend on the
    // tokens) and stay in flight across the token compaction
    uint4 ar[FS_SW][F16A ? 1 : 2];
#pragma unroll
    for (int i = 0; i < FS_SW; ++i) {
        const int k = k0 + 32 * (wave + 16 * i) + 8 * c;
        const int kk = k < k1 ? k : k0; // a valid address; the values are zeroed
        if (F16A) {
            ar[i][0] = *(gu4_t *)((gf16_t *)e.a + (size_t)jr * K + kk);
        } else {
            gf32_t *src = (gf32_t *)e.a + (size_t)jr * K + kk;
            ar[i][0] = __builtin_bit_cast(uint4, *(gf4_t *)src);
            ar[i][F16A ? 0 : 1] = __builtin_bit_cast(uint4, *(gf4_t *)(src + 4));
        }
    }
    // the adapter's tokens in token order (the batch fits one round: at most
    // LORA_FUSED_MAX_M tokens); LDS-only barriers leave the loads in flight
    const bool hit = idv == a;
    const unsigned long long m = __ballot(hit);
    if (lane == 0)
        wsum[wave] = __popcll(m);
    lds_barrier();
    int before = 0, count = 0;
#pragma unroll
    for (int w = 0; w < XPREP_TH / 64; ++w) {
        const int ws = wsum[w];
        before += w < wave ? ws : 0;
        count += ws;
    }
    if (hit)
        toks[before + __popcll(m & ((1ull << lane) - 1ull))] = threadIdx.x;
    lds_barrier();
    if (count == 0) // uniform
        return;
    constexpr int NA = F16A ? 2 : 3;
    bf16x8_t a1[FS_SW], a2[FS_SW], a3[FS_SW];
#pragma unroll
    for (int i = 0; i < FS_SW; ++i) {
        const bool live = k0 + 32 * (wave + 16 * i) + 8 * c < k1;
        float v[8];
        if (F16A) {
            const half8_t hv = __builtin_bit_cast(half8_t, ar[i][0]);
#pragma unroll
            for (int q = 0; q < 8; ++q)
                v[q] = live ? (float)hv[q] : 0.f;
        } else {
            const float4 f0 = __builtin_bit_cast(float4, ar[i][0]);
            const float4 f1 = __builtin_bit_cast(float4, ar[i][F16A ? 0 : 1]);
            const float w[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
#pragma unroll
            for (int q = 0; q < 8; ++q)
                v[q] = live ? w[q] : 0.f;
        }
        bf_split<NA>(v, a1[i], a2[i], a3[i]);
    }
    for (int tc = 0; tc < count; tc += 16) {
        const int ti = tc + r16;
        const int tok = toks[ti < count ? ti : 0];
        float xv[FS_SW][8];
#pragma unroll
        for (int i = 0; i < FS_SW; ++i) {
            const int k = k0 + 32 * (wave + 16 * i) + 8 * c;
            const bool live = k < k1;
            const size_t at = (size_t)tok * K + (live ? k : k0);
            const float4 f0 = *reinterpret_cast<const float4 *>(x + at);
            const float4 f1 = *reinterpret_cast<const float4 *>(x + at + 4);
            xv[i][0] = f0.x; xv[i][1] = f0.y; xv[i][2] = f0.z; xv[i][3] = f0.w;
            xv[i][4] = f1.x; xv[i][5] = f1.y; xv[i][6] = f1.z; xv[i][7] = f1.w;
            if (!live)
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    xv[i][q] = 0.f;
        }
        floatx4 P = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < FS_SW; ++i) {
            bf16x8_t b1, b2, b3;
            bf_split<3>(xv[i], b1, b2, b3);
            P = mfma_bf(b1, a1[i], P);
            P = mfma_bf(b1, a2[i], P);
            if (!F16A)
                P = mfma_bf(b1, a3[i], P);
            P = mfma_bf(b2, a1[i], P);
            P = mfma_bf(b2, a2[i], P);
            P = mfma_bf(b3, a1[i], P);
        }
        // D[token slot 4c + v][row r16] of every wave, summed over the waves
#pragma unroll
        for (int v = 0; v < 4; ++v)
            red[wave][4 * lane + v] = P[v];
        lds_barrier();
        if (threadIdx.x < 256) {
            float sum = 0.f;
#pragma unroll
            for (int w = 0; w < 16; ++w)
                sum += red[w][threadIdx.x];
            const int ln = threadIdx.x >> 2, v = threadIdx.x & 3;
            const int tj = tc + 4 * (ln >> 4) + v, row = jc + (ln & 15);
            if (tj < count && row < e.rank)
                pk[(size_t)toks[tj] * rmax + row] = sum;
        }
        lds_barrier();
    }
}

// Shrink workgroup wg (0-based past the xprep rows) of a fused launch.
REALM_DEV void lora_shrink_fused(const LoraGroupArgs &g, int wg)
{
    __shared__ int toks[LORA_FUSED_MAX_M];
    __shared__ int wsum[XPREP_TH / 64];
    __shared__ float red[16][256];
    // the token ids and the chunk entry: two independent loads
    const int idv = (int)threadIdx.x < g.M ? g.ids[threadIdx.x] : -1;
    const int p = (wg >= g.wg_start[1] ? 1 : 0) + (wg >= g.wg_start[2] ? 1 : 0) +
                  (wg >= g.wg_start[3] ? 1 : 0);
    const int local = wg - lora_pick(g.wg_start, p);
    const int ci = local / g.nparts, kp = local - ci * g.nparts;
    const LoraChunk ch = lora_pick(g.chunks, p)[ci];
    const int rmax = lora_pick(g.rmax, p);
    float *pk = lora_pick(g.u, p) + (size_t)kp * lora_pick(g.pstride, p);
    const int k0 = kp * LORA_FUSED_KP, k1 = min(g.K, k0 + LORA_FUSED_KP);
    const float *x = (const float *)g.x;
    if (ch.e.dtype)
        shrink_fused_body<true>(x, g.K, ch.e, ch.a, idv, pk, 16 * ch.rc, k0, k1, rmax, toks, wsum,
                                red);
    else
        shrink_fused_body<false>(x, g.K, ch.e, ch.a, idv, pk, 16 * ch.rc, k0, k1, rmax, toks, wsum,
                                 red);
}

// xprep for rows 0 .. rows - 1, the fused shrink past them
#define DEF_XPREP_LORA(NAME, FMT)                                                          \
    extern "C" __global__ __launch_bounds__(XPREP_TH) void realm_xprep_lora_##NAME(       \
        const void *x, int bf16, _Float16 *xh, _Float16 *xl, _Float16 *xm, float *tscale, \
        int M, int K, int KX, int rows, LoraGroupArgs g)                                   \
    {                                                                                      \
        if ((int)blockIdx.x < rows)                                                        \
            xprep<FMT, 0>(x, bf16, xh, xl, xm, tscale, M, K, KX);                          \
        else                                                                               \
            lora_shrink_fused(g, (int)blockIdx.x - rows);                                  \
    }                                                                                      \
    extern "C" __global__ __launch_bounds__(XPREP_TH) void realm_xprep_lora_##NAME##_o1(  \
        const void *x, int bf16, _Float16 *xh, _Float16 *xl, _Float16 *xm, float *tscale, \
        int M, int K, int KX, int rows, LoraGroupArgs g)                                   \
    {                                                                                      \
        if ((int)blockIdx.x < rows)                                                        \
            xprep<FMT, 1>(x, bf16, xh, xl, xm, tscale, M, K, KX);                          \
        else                                                                               \
            lora_shrink_fused(g, (int)blockIdx.x - rows);                                  \
    }
DEF_XPREP_LORA(q4k, FMT_Q4K)
DEF_XPREP_LORA(q6k, FMT_Q6K)
DEF_XPREP_LORA(q80, FMT_Q80)

// ------------------------------------------------------------ LoRA expand
//
// y[t][n] += scale_a * sum_j u[t][j] B_a[n][j] for the tokens t of adapter a
// (y already holds the base product).  Grid (adapter, group of RT 64-row
// tiles, 16-token chunk of the adapter's tokens); a wave sums the shrink's
// parts for its tokens once and sweeps 16 rows of each tile (RT = 8 for
// large grids; 4 or 2 give small adapter sets more workgroups):
// MFMA with A = u (token slots x rank, f32 split into f16 hi/lo), B = B_a^T
// (rank x rows, f16 exact or f32 split).  Every (t, n) belongs to one
// adapter, so the read-modify-write of y has no conflicts.
#define EXPAND_KK 2  // rank steps of 32 held in registers: ranks up to 64
// One pass of rank steps kk0 .. kk0 + EXPAND_KK - 1 for this wave's 16 rows of
// each of the workgroup's 8 row tiles.  FAST: f16 B with a rank that is a
// multiple of 8, read 8 ranks per 16-byte load; otherwise f32 B (split into
// f16 hi + lo) or f16 B element by element.  All loads of y and B are issued
// before the u loads, and no loaded value is used before those are issued
// too (a use right after a load makes the wave wait for it).
template <bool FAST, int RT>
REALM_DEV void expand_body(const float *__restrict__ u, const LoraEntry &e,
                           const int *__restrict__ toks, int count, int tc, float *__restrict__ y,
                           int N, int rmax, int nparts, int pstride)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r16 = lane & 15, c = lane >> 4;
    // loads read valid memory whatever the lane (rows past N read row N-1,
    // token slots past the adapter's tokens its first token, ranks past the
    // rank a valid group): such values only reach D entries that are never
    // stored, or are masked to zero where they would enter a sum
    const int ti = tc + r16;
    const int tok = toks[ti < count ? ti : 0];
    int toko[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int tj = tc + 4 * c + v;
        toko[v] = toks[tj < count ? tj : 0];
    }
    auto brow = [&](int rt) {
        return min((int)(blockIdx.y * RT + rt) * 64 + wave * 16 + r16, N - 1);
    };
    const int ksteps = (e.rank + 31) / 32;
    for (int kk0 = 0; kk0 < ksteps; kk0 += EXPAND_KK) {
        const int nkk = min(EXPAND_KK, ksteps - kk0); // rank steps of this pass (uniform)
        float yv[RT][4];
        half8_t bh[RT][EXPAND_KK], bl[RT][EXPAND_KK];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                yv[rt][v] = y[(size_t)toko[v] * N + brow(rt)];
        if constexpr (FAST) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int q2 = 0; q2 < EXPAND_KK; ++q2) {
                    const int j0 = 32 * (kk0 + q2) + 8 * c;
                    gf16_t *src = (gf16_t *)e.b + (size_t)brow(rt) * e.rank + min(j0, e.rank - 8);
                    bh[rt][q2] = __builtin_bit_cast(half8_t, *(gu4_t *)src);
                }
        }
        // this wave's A fragments (u of its 16 tokens, up to 64 ranks): the
        // sum of the shrink's K parts, in part order, loads before the first
        // add; rank steps past the adapter's rank are skipped (uniform)
        float us[EXPAND_KK][8];
#pragma unroll
        for (int q2 = 0; q2 < EXPAND_KK; ++q2) {
#pragma unroll
            for (int q = 0; q < 8; ++q)
                us[q2][q] = 0.f;
            if (q2 >= nkk)
                continue;
            const int j0 = 32 * (kk0 + q2) + 8 * c; // this lane's 8 ranks
            const int ju = min(j0, rmax - 8);
            float uv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            for (int g0 = 0; g0 < nparts; g0 += 8) {
                float4 p0[8], p1[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const int kp = min(g0 + q, nparts - 1);
                    const float4 *up = reinterpret_cast<const float4 *>(
                        u + (size_t)kp * pstride + (size_t)tok * rmax + ju);
                    p0[q] = up[0];
                    p1[q] = up[1];
                }
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    if (g0 + q < nparts) {
                        uv[0] += p0[q].x; uv[1] += p0[q].y; uv[2] += p0[q].z; uv[3] += p0[q].w;
                        uv[4] += p1[q].x; uv[5] += p1[q].y; uv[6] += p1[q].z; uv[7] += p1[q].w;
                    }
                }
            }
#pragma unroll
            for (int q = 0; q < 8; ++q)
                us[q2][q] = j0 + q < e.rank ? uv[q] : 0.f;
        }
        // u is in the activations' units (a down projection's input can
        // reach 1e7 and more): each token slot's values of this pass are
        // rescaled by an exact power of two 2^-eu so that their max lands in
        // [512, 1024) before the f16 hi/lo split, as xprep does for x; the
        // product is multiplied back by 2^eu.  The four lanes c = 0..3 of a
        // token slot r16 hold its ranks.
        float umax = 0.f;
#pragma unroll
        for (int q2 = 0; q2 < EXPAND_KK; ++q2)
#pragma unroll
            for (int q = 0; q < 8; ++q)
                umax = fmaxf(umax, fabsf(us[q2][q]));
        umax = fmaxf(umax, __shfl_xor(umax, 16, 64));
        umax = fmaxf(umax, __shfl_xor(umax, 32, 64));
        int eu = 0;
        if (umax > 0.f && __builtin_isfinite(umax)) {
            int ex;
            frexpf(umax, &ex);
            eu = max(ex - 10, -126); // 2^-eu and 2^eu stay normal floats
        }
        const float udown = ldexpf(1.f, -eu), uup = ldexpf(1.f, eu);
        half8_t ah[EXPAND_KK], al[EXPAND_KK];
#pragma unroll
        for (int q2 = 0; q2 < EXPAND_KK; ++q2)
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float vq = us[q2][q] * udown;
                const _Float16 h = (_Float16)vq;
                ah[q2][q] = h;
                al[q2][q] = (_Float16)(vq - (float)h);
            }
        // the scale of each D token slot 4c + v (held by lane 4c + v)
        float dup[4];
#pragma unroll
        for (int v = 0; v < 4; ++v)
            dup[v] = __shfl(uup, 4 * c + v, 64);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int q2 = 0; q2 < EXPAND_KK; ++q2) {
                const int j0 = 32 * (kk0 + q2) + 8 * c;
                if constexpr (FAST) { // ranks past the adapter's enter the sum as zero
#pragma unroll
                    for (int q = 0; q < 8; ++q)
                        bh[rt][q2][q] = j0 + q < e.rank ? bh[rt][q2][q] : (_Float16)0.f;
                } else {
#pragma unroll
                    for (int q = 0; q < 8; ++q) {
                        const float vv =
                            lora_elem(e.b, e.dtype, (size_t)brow(rt) * e.rank + min(j0 + q, e.rank - 1));
                        const float vm = j0 + q < e.rank ? vv : 0.f;
                        const _Float16 hq = (_Float16)vm;
                        bh[rt][q2][q] = hq;
                        bl[rt][q2][q] = (_Float16)(vm - (float)hq);
                    }
                }
            }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const int row = (blockIdx.y * RT + rt) * 64 + wave * 16 + r16;
            floatx4 P = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int q2 = 0; q2 < EXPAND_KK; ++q2) {
                P = mfma(ah[q2], bh[rt][q2], P);
                P = mfma(al[q2], bh[rt][q2], P);
                if (!FAST && !e.dtype)
                    P = mfma(ah[q2], bl[rt][q2], P);
            }
            // D[token slot 4c+v][row r16]
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int tj = tc + 4 * c + v;
                if (tj < count && row < N)
                    y[(size_t)toks[tj] * N + row] = yv[rt][v] + e.scale * (P[v] * dup[v]);
            }
        }
    }
}

// Grid: (adapter slots of all projections, groups of 512 rows of the
// longest projection, 16-token chunks).
template <int RT>
REALM_DEV void lora_expand(const LoraGroupArgs &g)
{
    __shared__ int toks[1024];
    __shared__ int count;
    __shared__ int wsum[4];
    const int p = lora_proj(g, blockIdx.x);
    const int a = blockIdx.x - lora_pick(g.a_start, p);
    const int N = lora_pick(g.N, p);
    if ((int)blockIdx.y * RT * 64 >= N) // a shorter projection of the group
        return;
    adapter_tokens(g.ids, g.M, a, toks, &count, wsum);
    const int tc = blockIdx.z * 16; // this workgroup's 16 tokens of the adapter
    if (tc >= count)
        return;
    const float *u = lora_pick(g.u, p);
    float *y = lora_pick(g.y, p);
    const int rmax = lora_pick(g.rmax, p), pstride = lora_pick(g.pstride, p);
    const LoraEntry e = lora_pick(g.table, p)[a];
    if (e.dtype && (e.rank & 7) == 0)
        expand_body<true, RT>(u, e, toks, count, tc, y, N, rmax, g.nparts, pstride);
    else
        expand_body<false, RT>(u, e, toks, count, tc, y, N, rmax, g.nparts, pstride);
}

// Row tiles per workgroup: 8 (realm_lora_expand), 4 or 2.
extern "C" __global__ __launch_bounds__(256) void realm_lora_expand(LoraGroupArgs g)
{
    lora_expand<8>(g);
}
extern "C" __global__ __launch_bounds__(256) void realm_lora_expand_rt4(LoraGroupArgs g)
{
    lora_expand<4>(g);
}
extern "C" __global__ __launch_bounds__(256) void realm_lora_expand_rt2(LoraGroupArgs g)
{
    lora_expand<2>(g);
}

#define DEF_SHRINK1(NAME, FMT, ORD, SUF)                                                   \
    extern "C" __global__ __launch_bounds__(256) void realm_lora_shrink_##NAME##_f32##SUF( \
        LoraGroupArgs g)                                                                   \
    {                                                                                      \
        lora_shrink<FMT, true, ORD>(g);                                                    \
    }                                                                                      \
    extern "C" __global__ __launch_bounds__(256) void realm_lora_shrink_##NAME##_bf16##SUF(\
        LoraGroupArgs g)                                                                   \
    {                                                                                      \
        lora_shrink<FMT, false, ORD>(g);                                                   \
    }
#define DEF_SHRINK(NAME, FMT) DEF_SHRINK1(NAME, FMT, 0, ) DEF_SHRINK1(NAME, FMT, 1, _o1)
DEF_SHRINK(q4k, FMT_Q4K)
DEF_SHRINK(q6k, FMT_Q6K)
DEF_SHRINK(q80, FMT_Q80)

// Decode GEMV, one token: y[n] = sum_k W[n,k] x[k] for resident Q4_K / Q6_K /
// Q8_0 weights in the device layout of common.h.
//
// Work decomposition: a row is cut into U "units" of 64 weights (Q4_K: one
// 32-byte qs group + the block header; Q6_K: one 48-byte ql/qh group + 4
// sub-scales + d; Q8_0: two 34-byte blocks).  LPR lanes share a row; lane l
// owns units l, l+LPR, ... (UPL of them) of every row it visits, and the wave
// handles 64/LPR row slots with R rows each per pass, grid-striding over
// passes.  x (f32) is staged once per workgroup in LDS and each lane keeps the
// per-unit sums of x it needs (Sx), so the Q4_K min term and the Q6_K / Q8_0
// offsets (-32, +128 bias) cost nothing per weight.  All R rows of a pass are
// loaded before any is consumed (memory-level parallelism), and each x value
// read from LDS is applied to R rows.
#include "common.h"

using namespace realm;

namespace {

template <int LPR>
struct Lanes {
    static constexpr int RPW = 64 / LPR; // row slots per wave
};

// Stage x[0..K) into LDS xs[0..KX), zero padding past K.
REALM_DEV void stage_x(float *xs, const float *__restrict__ x, int K, int KX)
{
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    float4 *xs4 = reinterpret_cast<float4 *>(xs);
    for (int i = threadIdx.x; i < KX / 4; i += blockDim.x)
        xs4[i] = (4 * i < K) ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    __syncthreads();
}

REALM_DEV float dot4(uint32_t w, float4 x, float acc)
{
    acc += ubyte0(w) * x.x;
    acc += ubyte1(w) * x.y;
    acc += ubyte2(w) * x.z;
    acc += ubyte3(w) * x.w;
    return acc;
}

REALM_DEV uint32_t word(const uint4 &v, int i)
{
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

REALM_DEV float4 lds4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

// ------------------------------------------------------------------- Q4_K

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

template <int LPR, int UPL, int R>
REALM_DEV void gemv_q4k(const uint8_t *__restrict__ hdr, const uint8_t *__restrict__ qs,
                        const float *__restrict__ x, float *__restrict__ y, int N, int K,
                        int nan_fb)
{
    extern __shared__ float xs[];
    const int U = K >> 6, B = K >> 8;
    stage_x(xs, x, K, K);
    const int lane = threadIdx.x & 63;
    const int slot = lane / LPR, l = lane % LPR;
    const int wpb = blockDim.x >> 6;
    const int gw = blockIdx.x * wpb + (threadIdx.x >> 6);
    const int nw = gridDim.x * wpb;

    float sxl[UPL], sxh[UPL];
#pragma unroll
    for (int j = 0; j < UPL; ++j) {
        int u = l + j * LPR;
        float a = 0.f, b = 0.f;
        if (u < U) {
            const float *xu = xs + 64 * u;
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                float4 v = lds4(xu + i), w = lds4(xu + 32 + i);
                a += (v.x + v.y) + (v.z + v.w);
                b += (w.x + w.y) + (w.z + w.w);
            }
        }
        sxl[j] = a;
        sxh[j] = b;
    }

    constexpr int RPP = Lanes<LPR>::RPW * R; // rows per pass per wave
    const int npass = (N + RPP - 1) / RPP;
    for (int p = gw; p < npass; p += nw) {
        const int r0 = p * RPP + slot * R;
        uint4 q0[R][UPL], q1[R][UPL], hd[R][UPL];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int j = 0; j < UPL; ++j) {
                int row = r0 + r, u = l + j * LPR;
                if (row < N && u < U) {
                    const uint8_t *qp = qs + (size_t)row * (K >> 1) + 32 * u;
                    q0[r][j] = ldg16(qp);
                    q1[r][j] = ldg16(qp + 16);
                    hd[r][j] = ldg16(hdr + ((size_t)row * B + (u >> 2)) * 16);
                } else {
                    q0[r][j] = q1[r][j] = hd[r][j] = make_uint4(0, 0, 0, 0);
                }
            }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
            acc[r] = 0.f;
#pragma unroll
        for (int j = 0; j < UPL; ++j) {
            int u = l + j * LPR;
            if (u < U) {
                const float *xu = xs + 64 * u;
                float dl[R], dh[R];
#pragma unroll
                for (int r = 0; r < R; ++r)
                    dl[r] = dh[r] = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    float4 xl = lds4(xu + 4 * i), xh = lds4(xu + 32 + 4 * i);
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        uint32_t w = word(i < 4 ? q0[r][j] : q1[r][j], i & 3);
                        dl[r] = dot4(w & 0x0F0F0F0Fu, xl, dl[r]);
                        dh[r] = dot4((w >> 4) & 0x0F0F0F0Fu, xh, dh[r]);
                    }
                }
                int g = u & 3;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float d = fix_scale(f16_bits_to_f32(hd[r][j].x), 0.00000006f, nan_fb);
                    float dm = fix_scale(f16_bits_to_f32(hd[r][j].x >> 16), 0.00000024f, nan_fb);
                    float sl, ml, sh, mh;
                    q4k_pair_rt(hd[r][j].y, hd[r][j].z, hd[r][j].w, g, sl, ml, sh, mh);
                    acc[r] += (d * sl) * dl[r] + (d * sh) * dh[r] -
                              ((dm * ml) * sxl[j] + (dm * mh) * sxh[j]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float v = group_sum<LPR>(acc[r]);
            int row = r0 + r;
            if (l == 0 && row < N)
                y[row] = v;
        }
    }
}

// ------------------------------------------------------------------- Q6_K

template <int LPR, int UPL, int R>
REALM_DEV void gemv_q6k(const uint8_t *__restrict__ dq, const int8_t *__restrict__ scq,
                        const uint8_t *__restrict__ qq, const float *__restrict__ x,
                        float *__restrict__ y, int N, int K, int nan_fb)
{
    extern __shared__ float xs[];
    const int U = K >> 6, B = K >> 8;
    stage_x(xs, x, K, K);
    const int lane = threadIdx.x & 63;
    const int slot = lane / LPR, l = lane % LPR;
    const int wpb = blockDim.x >> 6;
    const int gw = blockIdx.x * wpb + (threadIdx.x >> 6);
    const int nw = gridDim.x * wpb;

    // unit u: block u>>2, v = u&3, h = v>>1, is = v&1; element (t, j) at
    // x[256b + 128h + 16is + 32t + j].
    float sx[UPL][4];
#pragma unroll
    for (int j = 0; j < UPL; ++j) {
        int u = l + j * LPR;
#pragma unroll
        for (int t = 0; t < 4; ++t)
            sx[j][t] = 0.f;
        if (u < U) {
            int v = u & 3;
            const float *xu = xs + 256 * (u >> 2) + 128 * (v >> 1) + 16 * (v & 1);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                float s = 0.f;
#pragma unroll
                for (int i = 0; i < 16; i += 4) {
                    float4 a = lds4(xu + 32 * t + i);
                    s += (a.x + a.y) + (a.z + a.w);
                }
                sx[j][t] = s;
            }
        }
    }

    constexpr int RPP = Lanes<LPR>::RPW * R;
    const int npass = (N + RPP - 1) / RPP;
    for (int p = gw; p < npass; p += nw) {
        const int r0 = p * RPP + slot * R;
        uint4 qa[R][UPL], qb[R][UPL], qh[R][UPL];
        uint32_t scw[R][UPL], dw[R][UPL];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int j = 0; j < UPL; ++j) {
                int row = r0 + r, u = l + j * LPR;
                if (row < N && u < U) {
                    const uint8_t *qp = qq + ((size_t)row * B * 4 + u) * 48;
                    qa[r][j] = ldg16(qp);
                    qb[r][j] = ldg16(qp + 16);
                    qh[r][j] = ldg16(qp + 32);
                    size_t blk = (size_t)row * B + (u >> 2);
                    scw[r][j] = ldg4(scq + blk * 16 + 4 * (u & 3));
                    dw[r][j] = *reinterpret_cast<const uint16_t *>(dq + blk * 2);
                } else {
                    qa[r][j] = qb[r][j] = qh[r][j] = make_uint4(0, 0, 0, 0);
                    scw[r][j] = dw[r][j] = 0;
                }
            }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
            acc[r] = 0.f;
#pragma unroll
        for (int j = 0; j < UPL; ++j) {
            int u = l + j * LPR;
            if (u < U) {
                int v = u & 3;
                const float *xu = xs + 256 * (u >> 2) + 128 * (v >> 1) + 16 * (v & 1);
                float pt[R][4];
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        pt[r][t] = 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float4 x0 = lds4(xu + 4 * i), x1 = lds4(xu + 32 + 4 * i);
                    float4 x2 = lds4(xu + 64 + 4 * i), x3 = lds4(xu + 96 + 4 * i);
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        uint32_t a = word(qa[r][j], i), b = word(qb[r][j], i);
                        uint32_t h = word(qh[r][j], i);
                        uint32_t v0 = (a & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
                        uint32_t v1 = (b & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
                        uint32_t v2 = ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
                        uint32_t v3 = ((b >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
                        pt[r][0] = dot4(v0, x0, pt[r][0]);
                        pt[r][1] = dot4(v1, x1, pt[r][1]);
                        pt[r][2] = dot4(v2, x2, pt[r][2]);
                        pt[r][3] = dot4(v3, x3, pt[r][3]);
                    }
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float d = fix_scale(f16_bits_to_f32(dw[r][j]), 0.00000006f, nan_fb);
                    uint32_t s = scw[r][j];
                    float part = 0.f;
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        float sc = (float)(int8_t)(s >> (8 * t));
                        part += sc * (pt[r][t] - 32.f * sx[j][t]);
                    }
                    acc[r] += d * part;
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float v = group_sum<LPR>(acc[r]);
            int row = r0 + r;
            if (l == 0 && row < N)
                y[row] = v;
        }
    }
}

// ------------------------------------------------------------------- Q8_0

template <int LPR, int UPL, int R>
REALM_DEV void gemv_q80(const uint8_t *__restrict__ dq, const int8_t *__restrict__ qq,
                        const float *__restrict__ x, float *__restrict__ y, int N, int K,
                        int KP)
{
    extern __shared__ float xs[];
    const int U = KP >> 6;
    stage_x(xs, x, K, KP);
    const int lane = threadIdx.x & 63;
    const int slot = lane / LPR, l = lane % LPR;
    const int wpb = blockDim.x >> 6;
    const int gw = blockIdx.x * wpb + (threadIdx.x >> 6);
    const int nw = gridDim.x * wpb;

    float s0[UPL], s1[UPL];
#pragma unroll
    for (int j = 0; j < UPL; ++j) {
        int u = l + j * LPR;
        float a = 0.f, b = 0.f;
        if (u < U) {
            const float *xu = xs + 64 * u;
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                float4 v = lds4(xu + i), w = lds4(xu + 32 + i);
                a += (v.x + v.y) + (v.z + v.w);
                b += (w.x + w.y) + (w.z + w.w);
            }
        }
        s0[j] = a;
        s1[j] = b;
    }

    constexpr int RPP = Lanes<LPR>::RPW * R;
    const int npass = (N + RPP - 1) / RPP;
    for (int p = gw; p < npass; p += nw) {
        const int r0 = p * RPP + slot * R;
        uint4 q[R][UPL][4];
        uint32_t dw[R][UPL];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int j = 0; j < UPL; ++j) {
                int row = r0 + r, u = l + j * LPR;
                if (row < N && u < U) {
                    const int8_t *qp = qq + (size_t)row * KP + 64 * u;
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        q[r][j][c] = ldg16(qp + 16 * c);
                    dw[r][j] = ldg4(dq + ((size_t)row * (KP >> 5) + 2 * u) * 2);
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        q[r][j][c] = make_uint4(0, 0, 0, 0);
                    dw[r][j] = 0;
                }
            }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
            acc[r] = 0.f;
#pragma unroll
        for (int j = 0; j < UPL; ++j) {
            int u = l + j * LPR;
            if (u < U) {
                const float *xu = xs + 64 * u;
                float pa[R], pb[R];
#pragma unroll
                for (int r = 0; r < R; ++r)
                    pa[r] = pb[r] = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    float4 xa = lds4(xu + 4 * i), xb = lds4(xu + 32 + 4 * i);
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        // bytes biased to unsigned: (q + 128)
                        uint32_t wa = word(q[r][j][i >> 2], i & 3) ^ 0x80808080u;
                        uint32_t wb = word(q[r][j][2 + (i >> 2)], i & 3) ^ 0x80808080u;
                        pa[r] = dot4(wa, xa, pa[r]);
                        pb[r] = dot4(wb, xb, pb[r]);
                    }
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float da = f16_bits_to_f32(dw[r][j]);
                    float db = f16_bits_to_f32(dw[r][j] >> 16);
                    acc[r] += da * (pa[r] - 128.f * s0[j]) + db * (pb[r] - 128.f * s1[j]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float v = group_sum<LPR>(acc[r]);
            int row = r0 + r;
            if (l == 0 && row < N)
                y[row] = v;
        }
    }
}

} // namespace

#define DEF_GEMV(LPR, UPL, R)                                                               \
    extern "C" __global__ __launch_bounds__(256) void realm_gemv_q4k_l##LPR##_u##UPL##_r##R( \
        const uint8_t *hdr, const uint8_t *qs, const float *x, float *y, int N, int K,        \
        int nan_fb)                                                                            \
    {                                                                                          \
        gemv_q4k<LPR, UPL, R>(hdr, qs, x, y, N, K, nan_fb);                                    \
    }                                                                                          \
    extern "C" __global__ __launch_bounds__(256) void realm_gemv_q6k_l##LPR##_u##UPL##_r##R( \
        const uint8_t *dq, const int8_t *scq, const uint8_t *qq, const float *x, float *y,    \
        int N, int K, int nan_fb)                                                              \
    {                                                                                          \
        gemv_q6k<LPR, UPL, R>(dq, scq, qq, x, y, N, K, nan_fb);                                \
    }                                                                                          \
    extern "C" __global__ __launch_bounds__(256) void realm_gemv_q80_l##LPR##_u##UPL##_r##R( \
        const uint8_t *dq, const int8_t *qq, const float *x, float *y, int N, int K, int KP)  \
    {                                                                                          \
        gemv_q80<LPR, UPL, R>(dq, qq, x, y, N, K, KP);                                         \
    }

// (lanes per row, units per lane, rows per pass) variants the host chooses from.
DEF_GEMV(16, 1, 1)
DEF_GEMV(16, 1, 2)
DEF_GEMV(16, 1, 4)
DEF_GEMV(32, 1, 1)
DEF_GEMV(32, 1, 2)
DEF_GEMV(32, 1, 4)
DEF_GEMV(32, 2, 1)
DEF_GEMV(32, 2, 2)
DEF_GEMV(64, 1, 1)
DEF_GEMV(64, 1, 2)
DEF_GEMV(64, 1, 4)
DEF_GEMV(64, 2, 1)
DEF_GEMV(64, 2, 2)
DEF_GEMV(64, 3, 1)
DEF_GEMV(64, 3, 2)
DEF_GEMV(64, 4, 1)
DEF_GEMV(64, 5, 1)
DEF_GEMV(64, 6, 1)
DEF_GEMV(64, 7, 1)
DEF_GEMV(64, 8, 1)

// Dense f32 GEMM behind GpuBackendTrait::matmul and the candle_matmul host
// functions: C[m,n] = sum_k A[m,k] B'[k,n] with B' = B ([k,n] row-major) or,
// for the transposed form, B' = B^T with B stored [n,k].
//
// On v_mfma_f32_32x32x2_f32: f32 products and f32 sums, so results differ
// from a CPU f32 loop only in the order of the additions.  Lane l = r32 + 32h
// supplies A[r32][h] and B[h][r32]; element v of its result is
// D[8(v/4) + 4h + v%4][r32] (checked on the GPU).
//
//  * A workgroup (4 waves) owns TMR rows x 128 columns of C.  TMR = 128:
//    2 x 2 waves of 64 x 64 (four 32 x 32 MFMA tiles each); TMR = 64 or 32
//    (skinny products: rows past M would be wasted MFMA work and loads):
//    1 x 4 waves of TMR x 32.
//  * Launches with few tiles (skinny products) split K over blockIdx.z.
//  * K goes in slices of 16 (64 for the skinny tiles), staged in LDS
//    k-major (As[k][m], Bs[k][n], rows padded), double buffered: the next
//    slice's global loads are in flight while the current one is
//    multiplied, one barrier per slice.  Out-of-range elements load as zero
//    (clamped address, select), so edges need no branches around loads.
#include "common.h"

namespace {
constexpr int TN = 128;
typedef float floatx16 __attribute__((ext_vector_type(16)));
}

// blockIdx.z = K split: the workgroup sums k in [z K/ks, (z+1) K/ks) and,
// with ks > 1, writes its part to part + z M N (realm_dense_reduce adds the
// parts in split order).
template <int TMR, int KT>
__device__ __forceinline__ void dense_f32(const float *__restrict__ A, const float *__restrict__ B,
                                          float *__restrict__ C, int M, int N, int K, int b_trans,
                                          int ks, float *__restrict__ part)
{
    constexpr int WMW = TMR == 128 ? 2 : 1;         // waves along M
    constexpr int WR = TMR / WMW, WC = TN * WMW / 4; // a wave's rows, columns
    constexpr int TI = WR / 32, TJ = WC / 32;        // its 32 x 32 MFMA tiles
    // a slice is KT positions of k; thread t stages k = t % KT of rows
    // t / KT + RS i (A, B^T): RA rows of A, RB of B per thread and slice
    constexpr int RS = 256 / KT, RA = TMR / RS, RB = TN / RS;
    // LDS rows padded so that the k-major stores of 64-position slices (64
    // lanes at consecutive k) fall in distinct banks
    constexpr int LPA = KT == 64 ? TMR + 1 : TMR + 4, LPB = KT == 64 ? TN + 1 : TN + 4;
    __shared__ float As[2][KT][LPA];
    __shared__ float Bs[2][KT][LPB];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r32 = lane & 31, h = lane >> 5;
    const int wm = wave % WMW, wn = wave / WMW;
    const int m0 = blockIdx.y * TMR, n0 = blockIdx.x * TN;
    const int kb = (int)(((long long)K * blockIdx.z) / ks), ke = (int)(((long long)K * (blockIdx.z + 1)) / ks);
    float *const out = ks > 1 ? part + (size_t)blockIdx.z * M * N : C;

    // global -> register staging of one slice.  A (and B^T): thread t reads
    // k = t % KT of rows t / KT + RS i, 4 KT contiguous bytes per row; B:
    // column t % 128 of slice rows t / 128 + 2i.
    const int kt = tid % KT, rb0 = tid / KT;
    float ra[RA], rb[RB];
    auto load_slice = [&](int k0) {
        const int ka = k0 + kt;
        const bool kin = ka < ke;
        const int kc = kin ? ka : ke - 1;
#pragma unroll
        for (int i = 0; i < RA; ++i) {
            const int m = m0 + rb0 + RS * i;
            const float v = A[(size_t)min(m, M - 1) * K + kc];
            ra[i] = (kin && m < M) ? v : 0.f;
        }
        if (b_trans) {
#pragma unroll
            for (int i = 0; i < RB; ++i) {
                const int n = n0 + rb0 + RS * i;
                const float v = B[(size_t)min(n, N - 1) * K + kc];
                rb[i] = (kin && n < N) ? v : 0.f;
            }
        } else {
            const int n = n0 + (tid & 127);
            const int ncl = min(n, N - 1);
#pragma unroll
            for (int i = 0; i < RB; ++i) {
                const int k = k0 + (tid >> 7) + 2 * i;
                const float v = B[(size_t)min(k, ke - 1) * N + ncl];
                rb[i] = (k < ke && n < N) ? v : 0.f;
            }
        }
    };
    auto store_slice = [&](int buf) {
#pragma unroll
        for (int i = 0; i < RA; ++i)
            As[buf][kt][rb0 + RS * i] = ra[i];
        if (b_trans) {
#pragma unroll
            for (int i = 0; i < RB; ++i)
                Bs[buf][kt][rb0 + RS * i] = rb[i];
        } else {
#pragma unroll
            for (int i = 0; i < RB; ++i)
                Bs[buf][(tid >> 7) + 2 * i][tid & 127] = rb[i];
        }
    };

    floatx16 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                acc[i][j][e] = 0.f;

    load_slice(kb);
    store_slice(0);
    __syncthreads();
    int cur = 0;
    for (int k0 = kb; k0 < ke; k0 += KT) {
        const bool more = k0 + KT < ke;
        if (more)
            load_slice(k0 + KT);
#pragma unroll
        for (int s = 0; s < KT / 2; ++s) {
            const int k = 2 * s + h;
            float a[TI], b[TJ];
#pragma unroll
            for (int i = 0; i < TI; ++i)
                a[i] = As[cur][k][wm * WR + 32 * i + r32];
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                b[j] = Bs[cur][k][wn * WC + 32 * j + r32];
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (more)
            store_slice(cur ^ 1); // the other buffer: every wave finished it last slice
        __syncthreads();
        cur ^= 1;
    }

#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int m = m0 + wm * WR + 32 * i + 8 * (v >> 2) + 4 * h + (v & 3);
                const int n = n0 + wn * WC + 32 * j + r32;
                if (m < M && n < N)
                    out[(size_t)m * N + n] = acc[i][j][v];
            }
}

// the skinny tiles take 64-position K slices: four times the bytes in flight
// per workgroup, which a product that streams B once needs
#define DENSE_F32(NAME, TMR, KT)                                                           \
    extern "C" __global__ __launch_bounds__(256) void NAME(                                \
        const float *__restrict__ A, const float *__restrict__ B, float *__restrict__ C,   \
        int M, int N, int K, int b_trans, int ks, float *__restrict__ part)                \
    {                                                                                      \
        dense_f32<TMR, KT>(A, B, C, M, N, K, b_trans, ks, part);                           \
    }
DENSE_F32(realm_dense_f32, 128, 16)
DENSE_F32(realm_dense_f32_m64, 64, 16)
DENSE_F32(realm_dense_f32_m32, 32, 16)

// C = the sum of the ks parts, in split order (deterministic)
extern "C" __global__ __launch_bounds__(256) void realm_dense_reduce(const float *__restrict__ part,
                                                                     float *__restrict__ C,
                                                                     long long n, int ks)
{
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n)
        return;
    // the parts' loads 8 at a time (one memory round trip per 8 parts)
    float s = 0.f;
    for (int z0 = 0; z0 < ks; z0 += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (z0 + u < ks)
                v[u] = part[(size_t)(z0 + u) * n + i];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (z0 + u < ks)
                s = z0 + u == 0 ? v[u] : s + v[u];
    }
    C[i] = s;
}

// out[i] = v for i < n (a kernel node, where a memset node would otherwise
// be recorded into a captured graph)
extern "C" __global__ __launch_bounds__(256) void realm_fill_f32(float *__restrict__ out,
                                                                 long long n, float v)
{
    const long long stride = (long long)gridDim.x * 256;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
        out[i] = v;
}

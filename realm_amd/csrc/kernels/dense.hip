// Dense f32 GEMM behind GpuBackendTrait::matmul and the candle_matmul host
// functions: C[m,n] = sum_k A[m,k] B'[k,n] with B' = B ([k,n] row-major) or,
// for the transposed form, B' = B^T with B stored [n,k].  f32 FMA on VALU,
// 64x64 tiles, 16-deep K slices staged in LDS, 4x4 outputs per thread.
#include "common.h"

namespace {
constexpr int TILE = 64, KT = 16;
}

extern "C" __global__ __launch_bounds__(256) void realm_dense_f32(
    const float *__restrict__ A, const float *__restrict__ B, float *__restrict__ C, int M,
    int N, int K, int b_trans)
{
    __shared__ float As[KT][TILE + 4];
    __shared__ float Bs[KT][TILE + 4];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int m0 = blockIdx.y * TILE, n0 = blockIdx.x * TILE;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += KT) {
        // 64x16 slice of A and 16x64 slice of B': 1024 elements each, 4 per thread
        for (int e = threadIdx.x; e < TILE * KT; e += 256) {
            int r = e / KT, kk = e % KT; // A: row r, column k0+kk
            int gm = m0 + r, gk = k0 + kk;
            As[kk][r] = (gm < M && gk < K) ? A[(size_t)gm * K + gk] : 0.f;
            float bv;
            if (b_trans) {
                int gn = n0 + r; // B[n][k]
                bv = (gn < N && gk < K) ? B[(size_t)gn * K + gk] : 0.f;
                Bs[kk][r] = bv;
            } else {
                int kk2 = e / TILE, c = e % TILE; // B[k][n]
                int gk2 = k0 + kk2, gn = n0 + c;
                bv = (gk2 < K && gn < N) ? B[(size_t)gk2 * N + gn] : 0.f;
                Bs[kk2][c] = bv;
            }
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < KT; ++kk) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                a[i] = As[kk][ty + 16 * i];
                b[i] = Bs[kk][tx + 16 * i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] += a[i] * b[j];
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int gm = m0 + ty + 16 * i, gn = n0 + tx + 16 * j;
            if (gm < M && gn < N)
                C[(size_t)gm * N + gn] = acc[i][j];
        }
}

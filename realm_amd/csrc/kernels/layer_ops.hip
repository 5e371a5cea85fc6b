// The element-wise operations of realm_forward_layer around the quantized
// products (crates/realm-runtime/src/memory64_host.rs:2059-2458), on f32
// activations resident on the device:
//   * RMSNorm, y = x / sqrt(mean(x^2) + eps) * w per row, as candle-nn's
//     ops::rms_norm that CandleNeuralOpsBackend::rms_norm calls
//     (crates/realm-compute-cpu/src/candle_neural_ops_backend.rs:32-60),
//     optionally fused with the residual add before it (h = x + r, written
//     out, then normed: memory64_host.rs:2318-2324 followed by :2337);
//   * SwiGLU, out = (g * (1 / (1 + exp(-g)))) * up (memory64_host.rs:
//     2419-2425), the operation order of the reference.
// Both are HBM-bound: vector loads and stores, one pass over each input.
#include "common.h"

namespace {

REALM_DEV float wave_sum(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        v += __shfl_xor(v, off, 64);
    return v;
}

// One workgroup of 256 threads per row; `hidden` is a multiple of 4 (the
// host checks), rows are read with float4 loads.  With `res` set, the row is
// h = x + res (written to `sum` when not null) before the norm.
__device__ void rms_norm_row(const float *__restrict__ x, const float *__restrict__ res,
                             const float *__restrict__ w, float eps, int hidden,
                             float *__restrict__ sum, float *__restrict__ y)
{
    __shared__ float partial[4];
    const size_t row = blockIdx.x;
    const float4 *xr = reinterpret_cast<const float4 *>(x + row * hidden);
    const float4 *rr = res ? reinterpret_cast<const float4 *>(res + row * hidden) : nullptr;
    const int n4 = hidden >> 2;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n4; i += 256) {
        float4 v = xr[i];
        if (rr) {
            const float4 r = rr[i];
            v.x += r.x; v.y += r.y; v.z += r.z; v.w += r.w;
            if (sum)
                reinterpret_cast<float4 *>(sum + row * hidden)[i] = v;
        }
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0)
        partial[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = partial[0] + partial[1] + partial[2] + partial[3];
    const float inv = 1.f / sqrtf(total / (float)hidden + eps);
    const float4 *wr = reinterpret_cast<const float4 *>(w);
    float4 *yr = reinterpret_cast<float4 *>(y + row * hidden);
    // the second pass re-reads the row from cache (its first pass just
    // brought it in), so HBM sees each input once
    for (int i = threadIdx.x; i < n4; i += 256) {
        float4 v = xr[i];
        if (rr) {
            const float4 r = rr[i];
            v.x += r.x; v.y += r.y; v.z += r.z; v.w += r.w;
        }
        const float4 g = wr[i];
        yr[i] = make_float4(v.x * inv * g.x, v.y * inv * g.y, v.z * inv * g.z, v.w * inv * g.w);
    }
}

} // namespace

extern "C" __global__ __launch_bounds__(256) void realm_rms_norm(
    const float *x, const float *res, const float *w, float eps, int hidden, float *sum, float *y)
{
    rms_norm_row(x, res, w, eps, hidden, sum, y);
}

// out[i] = silu(gate[i]) * up[i], float4 per thread over n4 vectors.
extern "C" __global__ __launch_bounds__(256) void realm_swiglu(const float4 *gate,
                                                               const float4 *up, size_t n4,
                                                               float4 *out)
{
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
        const float4 g = gate[i], u = up[i];
        float4 o;
        o.x = g.x * (1.f / (1.f + expf(-g.x))) * u.x;
        o.y = g.y * (1.f / (1.f + expf(-g.y))) * u.y;
        o.z = g.z * (1.f / (1.f + expf(-g.z))) * u.z;
        o.w = g.w * (1.f / (1.f + expf(-g.w))) * u.w;
        out[i] = o;
    }
}

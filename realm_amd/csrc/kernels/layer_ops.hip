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

// RoPE of realm's MultiHeadAttention::apply_rope (crates/realm-models/src/
// attention.rs:171-235), in place on x [seq][heads][head_dim]: interleaved
// pairs (i, i + 1), freq = 1 / theta^(i / head_dim), angle = (start + s) *
// freq, in the reference's f32 operation order.  One thread per pair.
namespace {

// (cos, sin) of the angle of pair (x_i, x_{i+1}) at absolute position pos,
// and the rotation by them: every rotation here goes through these two
// functions, so the fused and separate forms agree.
__device__ __forceinline__ float2 rope_cs(int i, int pos, int head_dim, float theta)
{
    const float freq = 1.0f / powf(theta, (float)i / (float)head_dim);
    const float angle = (float)pos * freq;
    return make_float2(cosf(angle), sinf(angle));
}
__device__ __forceinline__ float2 rope_apply(float2 a, float2 cs)
{
    return make_float2(a.x * cs.x - a.y * cs.y, a.x * cs.y + a.y * cs.x);
}
__device__ __forceinline__ float2 rope_rot(float2 a, int i, int pos, int head_dim, float theta)
{
    return rope_apply(a, rope_cs(i, pos, head_dim, theta));
}

// Pair p of x [seq][heads][head_dim] rotated in place.
__device__ __forceinline__ void rope_pair(float *x, size_t p, int heads, int head_dim, int start,
                                          float theta)
{
    const int half = head_dim >> 1;
    const int i = 2 * (int)(p % half);
    const int s = (int)(p / ((size_t)heads * half));
    float2 *v = reinterpret_cast<float2 *>(x) + p;
    *v = rope_rot(*v, i, start + s, head_dim, theta);
}

} // namespace

extern "C" __global__ __launch_bounds__(256) void realm_rope(float *x, int seq, int heads,
                                                             int head_dim, int start, float theta)
{
    const size_t pairs = (size_t)seq * heads * (head_dim >> 1);
    const size_t p = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (p < pairs)
        rope_pair(x, p, heads, head_dim, start, theta);
}

// Q and K of one layer in one launch: pairs of q first, then of k.
// (cos, sin) of the head_dim / 2 pair angles at position pos (the fused
// decode attention's rotations, once per step for every layer)
extern "C" __global__ __launch_bounds__(256) void realm_rope_table(float2 *cs, int head_dim,
                                                                   int pos, float theta)
{
    const int p = (int)(blockIdx.x * 256 + threadIdx.x);
    if (p < (head_dim >> 1))
        cs[p] = rope_cs(2 * p, pos, head_dim, theta);
}

// (cos, sin) of every pair angle at positions start .. start + seq - 1, cs[s][p]
// (a prefill chunk's rotations, once per call for every layer)
extern "C" __global__ __launch_bounds__(256) void realm_rope_table_seq(float2 *cs, int head_dim,
                                                                       int start, int seq,
                                                                       float theta)
{
    const int half = head_dim >> 1;
    const size_t p = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (p < (size_t)seq * half)
        cs[p] = rope_cs(2 * (int)(p % half), start + (int)(p / half), head_dim, theta);
}

// realm_rope_qk with the rotations read from a realm_rope_table_seq table of
// the same positions (no powf or sincos per pair)
extern "C" __global__ __launch_bounds__(256) void realm_rope_qk_tab(float *q, int q_heads, float *k,
                                                                    int k_heads, int seq,
                                                                    int head_dim, const float2 *cs)
{
    const int half = head_dim >> 1;
    const size_t pq = (size_t)seq * q_heads * half, pk = (size_t)seq * k_heads * half;
    const size_t p = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (p < pq) {
        const int i = (int)(p % half), t = (int)(p / ((size_t)q_heads * half));
        float2 *v = reinterpret_cast<float2 *>(q) + p;
        *v = rope_apply(*v, cs[(size_t)t * half + i]);
    } else if (p < pq + pk) {
        const size_t pp = p - pq;
        const int i = (int)(pp % half), t = (int)(pp / ((size_t)k_heads * half));
        float2 *v = reinterpret_cast<float2 *>(k) + pp;
        *v = rope_apply(*v, cs[(size_t)t * half + i]);
    }
}

extern "C" __global__ __launch_bounds__(256) void realm_rope_qk(float *q, int q_heads, float *k,
                                                                int k_heads, int seq, int head_dim,
                                                                int start, float theta)
{
    const size_t pq = (size_t)seq * q_heads * (head_dim >> 1);
    const size_t pk = (size_t)seq * k_heads * (head_dim >> 1);
    const size_t p = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (p < pq)
        rope_pair(q, p, q_heads, head_dim, start, theta);
    else if (p < pq + pk)
        rope_pair(k, p - pq, k_heads, head_dim, start, theta);
}

namespace {

REALM_DEV float wave_max(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

} // namespace

// Causal attention over a KV cache (MultiHeadAttention::compute_attention,
// attention.rs:300-380, with StandardAttention, crates/realm-runtime/src/
// attention/standard.rs:36-210): query token t (absolute position
// position + t) of head h attends to cached keys j <= position + t of KV
// head h / (heads / kv_heads); scores (q . k_j) / sqrt(head_dim), softmax
// with the maximum subtracted, weights normalized by their sum, output
// sum_j p_j v_j.  One workgroup of ATT_TH threads per (token, head); the
// scores of the visible keys live in dynamic LDS after q.  head_dim divides
// 256 (the host checks); the output sums run over head_dim x (ATT_TH /
// head_dim) threads, key slices summed in slice order.  The shuffle
// reduction of a key's partial dots stays inside its lpk-lane group
// (xor offsets below lpk), so groups never mix.
// Workgroup of the attention kernel: 16 waves, so that a (token, head)
// workgroup keeps 16 waves' key and value loads in flight.
#define ATT_TH 1024
#define ATT_NW (ATT_TH / 64)
extern "C" __global__ __launch_bounds__(ATT_TH) void realm_attention(
    const float *q, const float *kc, const float *vc, int kv_len, int position, int heads,
    int kv_heads, int head_dim, float scale, float *out)
{
    extern __shared__ float smem[];
    __shared__ float red[2 * ATT_NW];
    float *qs = smem;              // head_dim
    float *sc = smem + head_dim;   // visible keys
    float *acc = sc + kv_len;      // ATT_TH partial outputs
    const int t = blockIdx.x / heads, h = blockIdx.x % heads;
    const int kvh = h / (heads / kv_heads);
    const int kv_dim = kv_heads * head_dim;
    const int vis = min(kv_len, position + t + 1);
    const float *qr = q + ((size_t)t * heads + h) * head_dim;
    for (int d = threadIdx.x; d < head_dim; d += ATT_TH)
        qs[d] = qr[d];
    __syncthreads();
    // Scores: a key row is read by head_dim / 4 adjacent lanes, one float4
    // each (coalesced), and their partial dots meet by shuffles; a wave
    // covers 256 / head_dim keys per step, the workgroup ATT_NW times that.
    const int lpk = head_dim >> 2, kpw = 64 / lpk;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane % lpk, sub = lane / lpk;
    const float4 q4 = reinterpret_cast<const float4 *>(qs)[c];
    // 8 steps per round, every key load of the round issued before the
    // first is used (one memory round trip per round, not per step)
    float mx = -INFINITY;
    for (int base = wave * kpw; base < vis; base += 8 * ATT_NW * kpw) {
        float4 k4[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int jc = min(base + u * ATT_NW * kpw + sub, vis - 1);
            k4[u] = *reinterpret_cast<const float4 *>(kc + (size_t)jc * kv_dim +
                                                      (size_t)kvh * head_dim + 4 * c);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int j = base + u * ATT_NW * kpw + sub;
            float dot = q4.x * k4[u].x + q4.y * k4[u].y + q4.z * k4[u].z + q4.w * k4[u].w;
            for (int off = lpk >> 1; off > 0; off >>= 1)
                dot += __shfl_xor(dot, off, 64);
            const float sv = dot * scale;
            if (c == 0 && j < vis) {
                sc[j] = sv;
                mx = fmaxf(mx, sv);
            }
        }
    }
    __syncthreads(); // the exp pass below reads scores other waves wrote
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = red[0];
    for (int w = 1; w < ATT_NW; ++w)
        mx = fmaxf(mx, red[w]);
    // a non-finite score gets weight 0 (standard.rs:119-126); the max
    // ignores NaN and may be +Inf, which leaves every finite weight 0
    float sum = 0.f;
    for (int j = threadIdx.x; j < vis; j += ATT_TH) {
        const float e = __builtin_isfinite(sc[j]) ? expf(sc[j] - mx) : 0.f;
        sc[j] = e;
        sum += e;
    }
    sum = wave_sum(sum);
    if ((threadIdx.x & 63) == 0)
        red[ATT_NW + (threadIdx.x >> 6)] = sum;
    __syncthreads();
    sum = red[ATT_NW];
    for (int w = 1; w < ATT_NW; ++w)
        sum += red[ATT_NW + w];
    const float inv = sum > 0.f ? 1.f / sum : 1.f;
    const int parts = ATT_TH / head_dim;
    const int d = threadIdx.x % head_dim, part = threadIdx.x / head_dim;
    // weighted sum of V in key order (per slice), 8 keys per round with
    // their loads issued first; keys past the visible ones add zero
    float a = 0.f;
    for (int j0 = part; j0 < vis; j0 += 8 * parts) {
        float vv[8], pw[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int j = j0 + u * parts, jc = min(j, vis - 1);
            vv[u] = vc[(size_t)jc * kv_dim + (size_t)kvh * head_dim + d];
            pw[u] = j < vis ? sc[jc] * inv : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            a += pw[u] * vv[u];
    }
    acc[threadIdx.x] = a;
    __syncthreads();
    if (part == 0) {
        float o = acc[d];
        for (int p = 1; p < parts; ++p)
            o += acc[p * head_dim + d];
        out[((size_t)t * heads + h) * head_dim + d] = o;
    }
}

// Causal attention for many query tokens (prefill), tiled: one workgroup
// of 4 waves per (32 query tokens, head, key split) walks its visible keys
// in blocks of ATK (64, or 32 for head_dim 256), each block's K and V staged once in LDS for all 32
// queries (the one-workgroup-per-token kernel reads every visible key once
// per query).  Both products run on v_mfma_f32_16x16x4_f32 (f32 products
// and sums: results differ from a CPU f32 loop only in the order of the
// additions); lane l supplies A[l%16][l/16] and B[l/16][l%16], element v of
// its result is D[4(l/16) + v][l%16].
//  * S = Q K^T / sqrt(head_dim): wave w owns rows 16(w&1) and keys
//    (ATK/2)(w>>1) .. + ATK/2 - 1; its Q rows stay in registers for the whole
//    walk, a lane holding head_dim elements 16g + 4(l/16) .. + 3 of its row
//    per group g, read as float4 (K the same way from LDS), so the four
//    MFMA steps of a group take the float4's four components.
//  * Softmax online (thread t: row t / 8, keys (ATK/8)(t % 8) ..): the row's
//    running max m skips NaN scores (f32::max), a non-finite score gets
//    weight 0 (standard.rs:119-126), so an +Inf score zeroes every finite
//    weight and the row's output is 0; when the max grows the row's sum
//    and output are rescaled by exp(m_old - m_new).
//  * O += P V: wave w owns rows 16(w&1) and the 16-column tiles w>>1,
//    (w>>1) + 2, ...; P and V come from LDS.
// splits > 1: split s takes the keys [s chunk, (s+1) chunk) and writes the
// row's (m, l, unnormalized output) to part in realm_attention_split's
// layout, for realm_attention_combine; splits == 1 writes out directly.
// HD is 32, 64, 128 or 256 (the host checks, and that q and out are 16-byte
// aligned).
namespace {
typedef float floatx4 __attribute__((ext_vector_type(4)));
constexpr int ATQ = 32; // query rows per workgroup

// K and V rows k0 .. k0 + nk - 1 of one block into registers (rows past nk:
// K repeats row nk - 1, V is zero)
template <int HD, int NL>
__device__ __forceinline__ void att_load(const float *__restrict__ kc, const float *__restrict__ vc,
                                         int k0, int nk, int kvh, int kv_dim, int tid,
                                         float4 (&kr)[NL], float4 (&vr)[NL])
{
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const int f = tid + 256 * i, r = f / (HD / 4), c = f % (HD / 4);
        const size_t at = (size_t)(k0 + min(r, nk - 1)) * kv_dim + (size_t)kvh * HD + 4 * c;
        const float4 kk = *reinterpret_cast<const float4 *>(kc + at);
        const float4 vv = *reinterpret_cast<const float4 *>(vc + at);
        kr[i] = kk;
        vr[i] = r < nk ? vv : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

// ATK keys per block (32 or 64): each wave's S tile is 16 rows x ATK / 2
// keys (ATK / 32 MFMA tiles side by side), each softmax thread takes ATK / 8
// keys of its row
template <int HD, int ATK>
__device__ void attention_tiled(const float *__restrict__ q, const float *__restrict__ kc,
                                const float *__restrict__ vc, int seq, int kv_len, int position,
                                int heads, int kv_heads, float scale, int splits, int chunk,
                                float *__restrict__ out, float *__restrict__ part)
{
    constexpr int LK = HD + 4, LV = HD + 16, LP = ATK + 4; // padded LDS rows (floats)
    constexpr int NG = HD / 16;             // groups of 16 head_dim elements
    constexpr int NL = ATK * HD / 4 / 256;  // float4 of K (and of V) per thread and block
    constexpr int NT = HD / 32;             // 16 x 16 output tiles per wave
    constexpr int SJ = ATK / 32;            // 16 x 16 S tiles per wave
    constexpr int KPT = ATK / 8;            // keys per softmax thread
    __shared__ __align__(16) float Ks[ATK * LK];
    __shared__ __align__(16) float Vs[ATK * LV];
    __shared__ __align__(16) float Ps[ATQ * LP];
    __shared__ __align__(16) float Rs[ATQ];
    __shared__ float Ms[ATQ], Ls[ATQ];
    const int h = blockIdx.y, q0 = blockIdx.x * ATQ, sp = blockIdx.z;
    const int kvh = h / (heads / kv_heads), kv_dim = kv_heads * HD;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, lc = lane >> 4;
    const int nq = min(ATQ, seq - q0);
    // keys this workgroup walks: its split's, up to the last one any row of
    // the tile sees
    const int kb = (int)min((long long)sp * chunk, (long long)kv_len);
    const int kl = (int)min(min((long long)kb + chunk, (long long)kv_len),
                            (long long)position + q0 + nq);

    const int rw = 16 * (wave & 1), cw = (ATK / 2) * (wave >> 1);
    floatx4 qv[NG];
    {
        const int r = rw + lr;
        const float *qr = q + ((size_t)(q0 + min(r, nq - 1)) * heads + h) * HD + 4 * lc;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            const float4 v = *reinterpret_cast<const float4 *>(qr + 16 * g);
            qv[g] = r < nq ? floatx4{v.x, v.y, v.z, v.w} : floatx4{0.f, 0.f, 0.f, 0.f};
        }
    }
    floatx4 acc[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i)
        acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int qi = tid >> 3, kq = tid & 7;
    const int qpos = position + q0 + qi; // absolute position of softmax row qi
    float m = -INFINITY, l = 0.f;

    // global -> registers: float4 f = tid + 256 i of the block (row f / (HD/4));
    // keys past the walk weigh 0 and get zero V rows, so no 0 x (their
    // value) reaches the sums
    float4 kr[NL], vr[NL];
    if (kb < kl)
        att_load<HD, NL>(kc, vc, kb, min(ATK, kl - kb), kvh, kv_dim, tid, kr, vr);
    for (int k0 = kb; k0 < kl; k0 += ATK) {
        __syncthreads(); // every wave is done with the previous block's K, V and P
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int f = tid + 256 * i, r = f / (HD / 4), c = f % (HD / 4);
            *reinterpret_cast<float4 *>(Ks + r * LK + 4 * c) = kr[i];
            *reinterpret_cast<float4 *>(Vs + r * LV + 4 * c) = vr[i];
        }
        __syncthreads();
        if (k0 + ATK < kl) // the next block's loads fly during this one
            att_load<HD, NL>(kc, vc, k0 + ATK, min(ATK, kl - k0 - ATK), kvh, kv_dim, tid, kr, vr);
        // this wave's S tiles
        {
            floatx4 sv[SJ];
#pragma unroll
            for (int j = 0; j < SJ; ++j)
                sv[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int g = 0; g < NG; ++g)
#pragma unroll
                for (int j = 0; j < SJ; ++j) {
                    const float4 kk = *reinterpret_cast<const float4 *>(
                        Ks + (cw + 16 * j + lr) * LK + 4 * lc + 16 * g);
                    sv[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(qv[g][0], kk.x, sv[j], 0, 0, 0);
                    sv[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(qv[g][1], kk.y, sv[j], 0, 0, 0);
                    sv[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(qv[g][2], kk.z, sv[j], 0, 0, 0);
                    sv[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(qv[g][3], kk.w, sv[j], 0, 0, 0);
                }
#pragma unroll
            for (int j = 0; j < SJ; ++j)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    Ps[(rw + 4 * lc + v) * LP + cw + 16 * j + lr] = sv[j][v] * scale;
        }
        __syncthreads();
        // online softmax of row qi over keys KPT kq .. KPT kq + KPT - 1
        {
            float sv[KPT];
#pragma unroll
            for (int c4 = 0; c4 < KPT / 4; ++c4) {
                const float4 s4 = *reinterpret_cast<const float4 *>(Ps + qi * LP + KPT * kq + 4 * c4);
                sv[4 * c4] = s4.x;
                sv[4 * c4 + 1] = s4.y;
                sv[4 * c4 + 2] = s4.z;
                sv[4 * c4 + 3] = s4.w;
            }
            bool vis[KPT];
            float bmax = -INFINITY;
#pragma unroll
            for (int u = 0; u < KPT; ++u) {
                const int j = k0 + KPT * kq + u;
                vis[u] = qi < nq && j < kl && j <= qpos;
                if (vis[u])
                    bmax = fmaxf(bmax, sv[u]);
            }
#pragma unroll
            for (int off = 1; off < 8; off <<= 1)
                bmax = fmaxf(bmax, __shfl_xor(bmax, off, 64));
            const float mn = fmaxf(m, bmax);
            // rescale of what the row holds: 0 while it holds nothing
            const float rs = m == -INFINITY ? 0.f
                                            : (mn == INFINITY && m == INFINITY ? 1.f : expf(m - mn));
            float e[KPT], ps = 0.f;
#pragma unroll
            for (int u = 0; u < KPT; ++u) {
                e[u] = vis[u] && __builtin_isfinite(sv[u]) ? expf(sv[u] - mn) : 0.f;
                ps += e[u];
            }
#pragma unroll
            for (int c4 = 0; c4 < KPT / 4; ++c4)
                *reinterpret_cast<float4 *>(Ps + qi * LP + KPT * kq + 4 * c4) =
                    make_float4(e[4 * c4], e[4 * c4 + 1], e[4 * c4 + 2], e[4 * c4 + 3]);
#pragma unroll
            for (int off = 1; off < 8; off <<= 1)
                ps += __shfl_xor(ps, off, 64);
            l = l * rs + ps;
            m = mn;
            if (kq == 0)
                Rs[qi] = rs;
        }
        __syncthreads();
        // O = O rs + P V
        {
            const float4 r4 = *reinterpret_cast<const float4 *>(Rs + rw + 4 * lc);
#pragma unroll
            for (int i = 0; i < NT; ++i) {
                acc[i][0] *= r4.x;
                acc[i][1] *= r4.y;
                acc[i][2] *= r4.z;
                acc[i][3] *= r4.w;
            }
#pragma unroll
            for (int ks = 0; ks < ATK / 4; ++ks) {
                const float a = Ps[(rw + lr) * LP + 4 * ks + lc];
                const float *vp = Vs + (4 * ks + lc) * LV + lr;
#pragma unroll
                for (int i = 0; i < NT; ++i)
                    acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vp[16 * ((wave >> 1) + 2 * i)],
                                                                 acc[i], 0, 0, 0);
            }
        }
    }
    if (kq == 0) {
        Ms[qi] = m;
        Ls[qi] = l;
    }
    __syncthreads();
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int r = rw + 4 * lc + v;
        if (r >= nq)
            continue;
        const size_t th = (size_t)(q0 + r) * heads + h;
        if (splits == 1) {
            const float inv = Ls[r] > 0.f ? 1.f / Ls[r] : 0.f;
            float *orow = out + th * HD + lr;
#pragma unroll
            for (int i = 0; i < NT; ++i)
                orow[16 * ((wave >> 1) + 2 * i)] = acc[i][v] * inv;
        } else {
            float *pr = part + (th * splits + sp) * (HD + 2);
#pragma unroll
            for (int i = 0; i < NT; ++i)
                pr[2 + 16 * ((wave >> 1) + 2 * i) + lr] = acc[i][v];
        }
    }
    if (splits > 1 && tid < nq) {
        float *pr = part + (((size_t)(q0 + tid) * heads + h) * splits + sp) * (HD + 2);
        pr[0] = Ms[tid];
        pr[1] = Ls[tid];
    }
}
} // namespace

#define ATT_TILED(HD)                                                                          \
    extern "C" __global__ __launch_bounds__(256) void realm_attention_tiled_h##HD(             \
        const float *q, const float *kc, const float *vc, int seq, int kv_len, int position,  \
        int heads, int kv_heads, float scale, int splits, int chunk, float *out, float *part) \
    {                                                                                          \
        attention_tiled<HD, HD <= 128 ? 64 : 32>(q, kc, vc, seq, kv_len, position, heads,     \
                                                 kv_heads, scale, splits, chunk, out, part);   \
    }
ATT_TILED(32)
ATT_TILED(64)
ATT_TILED(128)
ATT_TILED(256)

// Residual add out[i] = a[i] + b[i] (CandleCpuBackend::add as
// realm_forward_layer uses it, memory64_host.rs:2452-2458), float4 per
// thread over n4 vectors.
extern "C" __global__ __launch_bounds__(256) void realm_add(const float4 *a, const float4 *b,
                                                            size_t n4, float4 *out)
{
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
        const float4 x = a[i], y = b[i];
        out[i] = make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w);
    }
}

// Split-K form of the attention for small grids (decode): workgroup
// (token, head, split s) takes the visible keys [s chunk, (s+1) chunk) and
// writes its partial max m_s, exp-sum l_s = sum exp(score - m_s) and
// unnormalized output acc_s = sum exp(score - m_s) v into
// part[((t * heads + h) * splits + s) * (head_dim + 2)]: (m, l, acc...).
// realm_attention_combine then forms m = max m_s, l = sum l_s e^(m_s - m),
// out = sum acc_s e^(m_s - m) / l, splits in order.  256 threads; the
// chunk's scores live in LDS.
// ROPE (the one-token decode step of the device layer): q arrives without
// its rotary embedding and the new key row (absolute position `position`)
// in k_new, also unrotated; both are rotated here by the (cos, sin) table of
// that position (realm_rope_table: rope_pair's values), and the workgroup of
// the first head of each KV group whose split holds that row writes the
// rotated row into the cache.  No workgroup of the launch reads that cache
// row: the row's keys come from k_new.
template <bool ROPE>
__device__ void attention_split(const float *q, float *kc, const float *vc, int kv_len,
                                int position, int heads, int kv_heads, int head_dim, float scale,
                                int splits, int chunk, float *part, const float *k_new,
                                const float2 *rcs)
{
    extern __shared__ float smem[];
    __shared__ float red[8];
    float *qs = smem, *sc = smem + head_dim, *acc = sc + chunk;
    const int s = blockIdx.x % splits, th = blockIdx.x / splits;
    const int t = th / heads, h = th % heads;
    const int kvh = h / (heads / kv_heads), kv_dim = kv_heads * head_dim;
    const int vis = min(kv_len, position + t + 1);
    const int j0 = s * chunk, j1 = min(vis, j0 + chunk);
    const int n = max(j1 - j0, 0);
    const float *qr = q + ((size_t)t * heads + h) * head_dim;
    // V rows of this thread's first VU keys (thread: column d, keys pp,
    // pp + parts, ...), loaded before anything else: their addresses depend
    // on nothing, so their latency hides behind the q and K phases
    constexpr int VU = 32;
    const int parts = 256 / head_dim;
    const int d = threadIdx.x % head_dim, pp = threadIdx.x / head_dim;
    float vv0[VU];
    if (n > 0) {
#pragma unroll
        for (int u = 0; u < VU; ++u) {
            const int jc = j0 + min(pp + u * parts, n - 1);
            vv0[u] = vc[(size_t)jc * kv_dim + (size_t)kvh * head_dim + d];
        }
    }
    if constexpr (ROPE) {
        const int half = head_dim >> 1;
        for (int pi = threadIdx.x; pi < half; pi += 256) { // (one token: t = 0)
            const int i = 2 * pi;
            const float2 r = rope_apply(make_float2(qr[i], qr[i + 1]), rcs[pi]);
            qs[i] = r.x;
            qs[i + 1] = r.y;
        }
        // the new key row: rotated into the cache once per KV head
        if (t == 0 && h % (heads / kv_heads) == 0 && position >= j0 && position < j1) {
            const float *kn = k_new + (size_t)kvh * head_dim;
            float *kw = kc + (size_t)position * kv_dim + (size_t)kvh * head_dim;
            for (int pi = threadIdx.x; pi < half; pi += 256) {
                const int i = 2 * pi;
                const float2 r = rope_apply(make_float2(kn[i], kn[i + 1]), rcs[pi]);
                kw[i] = r.x;
                kw[i + 1] = r.y;
            }
        }
    } else {
        for (int d = threadIdx.x; d < head_dim; d += 256)
            qs[d] = qr[d];
    }
    __syncthreads();
    const int lpk = head_dim >> 2, kpw = 64 / lpk;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane % lpk, sub = lane / lpk;
    const float4 q4 = reinterpret_cast<const float4 *>(qs)[c];
    float mx = -INFINITY;
    // the cached keys (ROPE: all but the step's new row, scored below)
    const int nc = ROPE ? max(min(j1, position) - j0, 0) : n;
    for (int base = wave * kpw; base < nc; base += 32 * kpw) {
        float4 k4[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int jc = j0 + min(base + u * 4 * kpw + sub, nc - 1);
            k4[u] = *reinterpret_cast<const float4 *>(kc + (size_t)jc * kv_dim +
                                                      (size_t)kvh * head_dim + 4 * c);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int jl = base + u * 4 * kpw + sub;
            float dot = q4.x * k4[u].x + q4.y * k4[u].y + q4.z * k4[u].z + q4.w * k4[u].w;
            for (int off = lpk >> 1; off > 0; off >>= 1)
                dot += __shfl_xor(dot, off, 64);
            const float sv = dot * scale;
            if (c == 0 && jl < nc) {
                sc[jl] = sv;
                mx = fmaxf(mx, sv);
            }
        }
    }
    if (ROPE && wave == 0 && position >= j0 && position < j1) {
        // the new row's score: its key from k_new, rotated; the same float4
        // grouping and shuffle order as the cached keys'
        float dot = 0.f;
        if (lane < lpk) {
            const float4 r = *reinterpret_cast<const float4 *>(
                k_new + (size_t)kvh * head_dim + 4 * lane);
            const float2 lo = rope_apply(make_float2(r.x, r.y), rcs[2 * lane]);
            const float2 hi = rope_apply(make_float2(r.z, r.w), rcs[2 * lane + 1]);
            dot = q4.x * lo.x + q4.y * lo.y + q4.z * hi.x + q4.w * hi.y;
        }
        for (int off = lpk >> 1; off > 0; off >>= 1)
            dot += __shfl_xor(dot, off, 64);
        if (lane == 0) {
            const float sv = dot * scale;
            sc[position - j0] = sv;
            mx = fmaxf(mx, sv);
        }
    }
    __syncthreads();
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float sum = 0.f; // non-finite scores: weight 0, as in realm_attention
    for (int j = threadIdx.x; j < n; j += 256) {
        const float e = __builtin_isfinite(sc[j]) ? expf(sc[j] - mx) : 0.f;
        sc[j] = e;
        sum += e;
    }
    sum = wave_sum(sum);
    if ((threadIdx.x & 63) == 0)
        red[4 + (threadIdx.x >> 6)] = sum;
    __syncthreads();
    sum = red[4] + red[5] + red[6] + red[7];
    // weighted sum of V in key order: the prefetched rows, then rounds of
    // VU loads issued together; keys past the visible ones add zero
    float a = 0.f;
    if (n > 0) {
        float pw[VU];
#pragma unroll
        for (int u = 0; u < VU; ++u) {
            const int jl = pp + u * parts;
            pw[u] = jl < n ? sc[min(jl, n - 1)] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < VU; ++u)
            a += pw[u] * vv0[u];
    }
    for (int jb = pp + VU * parts; jb < n; jb += VU * parts) {
        float vv[VU], pw[VU];
#pragma unroll
        for (int u = 0; u < VU; ++u) {
            const int jl = jb + u * parts, jc = j0 + min(jl, n - 1);
            vv[u] = vc[(size_t)jc * kv_dim + (size_t)kvh * head_dim + d];
            pw[u] = jl < n ? sc[min(jl, n - 1)] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < VU; ++u)
            a += pw[u] * vv[u];
    }
    acc[threadIdx.x] = a;
    __syncthreads();
    float *pr = part + ((size_t)th * splits + s) * (head_dim + 2);
    if (pp == 0) {
        float o = acc[d];
        for (int p = 1; p < parts; ++p)
            o += acc[p * head_dim + d];
        pr[2 + d] = o;
    }
    if (threadIdx.x == 0) {
        pr[0] = n > 0 ? mx : -INFINITY;
        pr[1] = n > 0 ? sum : 0.f;
    }
}

extern "C" __global__ __launch_bounds__(256) void realm_attention_split(
    const float *q, const float *kc, const float *vc, int kv_len, int position, int heads,
    int kv_heads, int head_dim, float scale, int splits, int chunk, float *part)
{
    attention_split<false>(q, const_cast<float *>(kc), vc, kv_len, position, heads, kv_heads,
                           head_dim, scale, splits, chunk, part, nullptr, nullptr);
}

extern "C" __global__ __launch_bounds__(256) void realm_attention_split_rope(
    const float *q, float *kc, const float *vc, int kv_len, int position, int heads,
    int kv_heads, int head_dim, float scale, int splits, int chunk, float *part,
    const float *k_new, const float2 *rope_cs_tab)
{
    attention_split<true>(q, kc, vc, kv_len, position, heads, kv_heads, head_dim, scale, splits,
                          chunk, part, k_new, rope_cs_tab);
}

// One workgroup of head_dim threads per (token, head).
extern "C" __global__ __launch_bounds__(256) void realm_attention_combine(
    const float *part, int splits, int head_dim, float *out)
{
    const int th = blockIdx.x, d = threadIdx.x;
    if (d >= head_dim)
        return;
    const float *pr = part + (size_t)th * splits * (head_dim + 2);
    float m = -INFINITY, l = 0.f, o = 0.f;
    if (splits <= 16) {
        // every split's (m, l, acc[d]) loaded at once (one memory round
        // trip; split s past `splits` reads the last one and is not used)
        float ms[16], ls[16], as[16];
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const float *p = pr + (size_t)min(s, splits - 1) * (head_dim + 2);
            ms[s] = p[0];
            ls[s] = p[1];
            as[s] = p[2 + d];
        }
#pragma unroll
        for (int s = 0; s < 16; ++s)
            if (s < splits)
                m = fmaxf(m, ms[s]);
#pragma unroll
        for (int s = 0; s < 16; ++s)
            if (s < splits) {
                const float w = ls[s] > 0.f ? expf(ms[s] - m) : 0.f;
                l += ls[s] * w;
                o += as[s] * w;
            }
    } else {
        for (int s = 0; s < splits; ++s)
            m = fmaxf(m, pr[(size_t)s * (head_dim + 2)]);
        for (int s = 0; s < splits; ++s) {
            const float *p = pr + (size_t)s * (head_dim + 2);
            const float w = p[1] > 0.f ? expf(p[0] - m) : 0.f;
            l += p[1] * w;
            o += p[2 + d] * w;
        }
    }
    out[(size_t)th * head_dim + d] = l > 0.f ? o / l : 0.f;
}

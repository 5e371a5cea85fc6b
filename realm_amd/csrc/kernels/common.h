// Device-side helpers shared by every gfx950 kernel of the quantized path.
//
// Device layout of a resident [N, K] matrix ("split streams", one region per
// field, each region 256-byte aligned; built by the repack kernels from the
// reference's packed blocks).  A row's quant bytes are cut into U = K/64
// "units" of 64 weights and stored plane-major: plane p of a row holds the
// p-th 16 bytes of every unit (row bytes [p*U*16 + u*16, +16)), so the 64
// lanes of a wave that own consecutive units read 1 KB contiguous per load.
//
//   Q4_K  hdr[N][K/256][16]  dword 0: d | dmin << 16 (as in the block);
//                            dwords 1..3: the 8 six-bit (scale, min) pairs of
//                            the block's 12 packed bytes (quant.rs:110-122),
//                            re-packed so that group g's four fields are the
//                            24 bits at bit 24g of the 96-bit field
//                            (sc[2g] | m[2g] << 6 | sc[2g+1] << 12 |
//                            m[2g+1] << 18): one funnel shift per lane.
//         qs [N][2][U][16]   unit u = qs group g = u%4 of block u/4 (32 bytes,
//                            halves in planes 0/1): byte j low nibble -> k =
//                            64u + j, high nibble -> k = 64u + 32 + j
//                            (crates/realm-core/src/quant.rs:155-184), the
//                            high nibble stored XOR 8: masked with 0xF0 it
//                            reads as the int8 16 * (q - 8).
//   Q6_K  d  [N][K/256]      f16 super-block scale
//         sc [N][K/256][16]  int8 sub-block scales regrouped per unit: unit v
//                            (v = 2h + is) holds sc[8h+is+2t], t = 0..3
//         q  [N][3][U][16]   unit u = (block u/4, v = u%4 = 2h + is): planes
//                            ql[64h+16is ..+16], ql[64h+32+16is ..+16],
//                            qh[32h+16is ..+16]; element (t, j) of the unit is
//                            k = 256b + 128h + 16is + 32t + j
//                            (quant.rs:393-451 regrouped).
//   Q8_0  d  [N][Kp/32]      f16 block scales
//         q  [N][4][U][16]   unit u = blocks 2u, 2u+1 (64 int8 quants, 16 per
//                            plane); Kp = K rounded up to 64, the padding is
//                            zero quants with zero scale.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define REALM_DEV static __device__ __forceinline__

namespace realm {

constexpr int QK_K = 256;
constexpr int Q4K_BLOCK_BYTES = 144;
constexpr int Q6K_BLOCK_BYTES = 210;
constexpr int Q80_BLOCK_BYTES = 34;

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also
// makes the wave wait for every global load it has in flight, which would
// stall the weight loads a kernel issues ahead of its first barrier.
REALM_DEV void lds_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

REALM_DEV float f16_bits_to_f32(uint32_t h)
{
    // v_cvt_f32_f16: exact, f16 subnormals preserved (f16 denormal mode is on).
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xFFFFu));
}

// crates/realm-core/src/quant.rs:110-122, for a pair of indices (2g, 2g+1),
// from the 12 scale bytes held as three dwords s0 (bytes 0..3), s1 (4..7),
// s2 (8..11).  Returns sc/m for j = 2g (lo) and j = 2g+1 (hi).
REALM_DEV void q4k_scale_min_pair(uint32_t s0, uint32_t s1, uint32_t s2, int g,
                                  uint32_t &sc_lo, uint32_t &m_lo,
                                  uint32_t &sc_hi, uint32_t &m_hi)
{
    // byte j of the 12 scales
    auto byte = [&](int j) -> uint32_t {
        uint32_t w = j < 4 ? s0 : (j < 8 ? s1 : s2);
        return (w >> (8 * (j & 3))) & 0xFFu;
    };
    auto get = [&](int j, uint32_t &sc, uint32_t &m) {
        if (j < 4) {
            sc = byte(j) & 63u;
            m = byte(j + 4) & 63u;
        } else {
            sc = (byte(j + 4) & 0xFu) | ((byte(j - 4) >> 6) << 4);
            m = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
        }
    };
    get(2 * g, sc_lo, m_lo);
    get(2 * g + 1, sc_hi, m_hi);
}

// The 24-bit (scale, min) field of Q4_K group g (0..3) from device header
// dwords h1..h3 (see the layout above).
REALM_DEV uint32_t q4k_dev_pair(uint32_t h1, uint32_t h2, uint32_t h3, int g)
{
    const uint32_t lo = g < 2 ? h1 : (g == 2 ? h2 : h3);
    const uint32_t hi = g < 2 ? h2 : h3;
    const uint32_t sh = (uint32_t)(24 * g) & 31u;
    return (uint32_t)((((uint64_t)hi << 32) | lo) >> sh);
}

// fused.rs NaN/Inf scale replacement (crates/realm-compute-cpu/src/
// fused.rs:276-285): applied only when the caller asks for fused.rs semantics.
REALM_DEV float fix_scale(float v, float fallback, int enable)
{
    return (enable && !__builtin_isfinite(v)) ? fallback : v;
}

// Sum over the lanes of an aligned group of `width` lanes (power of two <= 64),
// result valid in every lane of the group.
template <int WIDTH>
REALM_DEV float group_sum(float v)
{
#pragma unroll
    for (int off = WIDTH / 2; off > 0; off >>= 1)
        v += __shfl_xor(v, off, 64);
    return v;
}

REALM_DEV uint4 ldg16(const void *p) { return *reinterpret_cast<const uint4 *>(p); }
REALM_DEV uint2 ldg8(const void *p) { return *reinterpret_cast<const uint2 *>(p); }
REALM_DEV uint32_t ldg4(const void *p) { return *reinterpret_cast<const uint32_t *>(p); }

// Byte e of a dword as float (selected as v_cvt_f32_ubyte{0..3}).
REALM_DEV float ubyte0(uint32_t w) { return (float)(w & 0xFFu); }
REALM_DEV float ubyte1(uint32_t w) { return (float)((w >> 8) & 0xFFu); }
REALM_DEV float ubyte2(uint32_t w) { return (float)((w >> 16) & 0xFFu); }
REALM_DEV float ubyte3(uint32_t w) { return (float)(w >> 24); }

} // namespace realm

// MFMA helpers shared by the batched kernels (gemm.hip, gemm_tiled.hip):
// f16 fragment types, the k-slot order xprep writes and the kernels read, and
// the v_mfma_f32_16x16x32_f16 wrapper.
#pragma once

#include "common.h"
#include "exact.h"

#define FMT_Q4K 0
#define FMT_Q6K 1
#define FMT_Q80 2

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace realm_mfma {

using namespace realm;

// Slot order inside an 8-slot group: nibble/byte pairs (0,2),(1,3),(4,6),(5,7)
// come out of one mask each, so slot e holds element PI[e] of its window.
REALM_DEV int pi8(int e) { return (e & 4) | ((e & 1) << 1) | ((e >> 1) & 1); }

// Activation slot orders.  xprep writes token t's activations as f16 at
// positions p = 8 pg + e (position group pg, slot e); the element behind slot
// e of pg is x[t][kwin(pg) + (w & 3) + kgap * (w >> 2)] with w = pi8(e).
//  ORD 0 (v_mfma_f32_16x16x32_f16, gemm.hip): pg = 32b + 4i + c is k-step i
//         (32 k) of 256-block b, lane group c; 8 consecutive k per window.
//  ORD 1 (v_mfma_f32_32x32x16_f16, gemm_tiled.hip): pg = 32b + 2s + h is
//         k-step s (16 k) of block b, lane half h; a window is 4 k plus the 4
//         k one sub-block (Q4_K: 32 k) or two (Q6_K: 64 k) further, i.e. the
//         low and high nibbles of one weight dword.
// Either way a lane's weights for a k-step are contiguous bytes of its row.
template <int FMT, int ORD>
REALM_DEV int kwin(int pg)
{
    if (FMT == FMT_Q80) {
        if (ORD == 0)
            return 8 * pg;
        // k-step s = 2i + t of block b, lane half h: 8 k of the 16 that
        // load i of gemm_tiled.hip brings (plane i/2 of unit 2(i&1) + h), so
        // that a lane's weight loads are 16 bytes and a row's two lanes read
        // 32 contiguous bytes
        const int b = pg >> 5, s = (pg >> 1) & 15, h = pg & 1, i = s >> 1;
        return 256 * b + 64 * (2 * (i & 1) + h) + 16 * (i >> 1) + 8 * (s & 1);
    }
    if (ORD == 0) {
        const int b = pg >> 5, i = (pg >> 2) & 7, c = pg & 3;
        if (FMT == FMT_Q4K)
            return 256 * b + 64 * c + 32 * (i >> 2) + 8 * (i & 3);
        return 256 * b + 128 * (c >> 1) + 16 * (c & 1) + 32 * (i >> 1) + 8 * (i & 1);
    }
    const int b = pg >> 5, s = (pg >> 1) & 15, h = pg & 1;
    if (FMT == FMT_Q4K) // unit 2h + s/8 of the block, plane (s/4)&1, dword s&3
        return 256 * b + 64 * (2 * h + (s >> 3)) + 16 * ((s >> 2) & 1) + 4 * (s & 3);
    // unit 2h + is (is = s/8), ql dword (s/2)&3 of plane A (s even: t = 0, 2)
    // or B (s odd: t = 1, 3)
    return 256 * b + 128 * h + 16 * (s >> 3) + 32 * (s & 1) + 4 * ((s >> 1) & 3);
}
template <int FMT, int ORD>
constexpr int kgap()
{
    return (ORD == 0 || FMT == FMT_Q80) ? 4 : (FMT == FMT_Q4K ? 32 : 64);
}
template <int FMT>
REALM_DEV int kwin(int pg) { return kwin<FMT, 0>(pg); }

REALM_DEV half2_t h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
REALM_DEV uint32_t u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }
REALM_DEV half8_t h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d)
{
    uint4 v = make_uint4(a, b, c, d);
    return __builtin_bit_cast(half8_t, v);
}
REALM_DEV half8_t ld_h8(const _Float16 *p) { return __builtin_bit_cast(half8_t, ldg16(p)); }
REALM_DEV half2_t splat2(float v)
{
    _Float16 h = (_Float16)v;
    half2_t r = {h, h};
    return r;
}

// Pointers read from device tables (adapter factors): cast to the global
// address space so that their loads are global loads (a flat load also
// counts against the LDS/scalar counter and makes every LDS wait wait for it
// too).
typedef __attribute__((address_space(1))) const _Float16 gf16_t;
typedef __attribute__((address_space(1))) const float gf32_t;
typedef __attribute__((address_space(1))) const uint4 gu4_t;
typedef __attribute__((address_space(1))) const uint2 gu2_t;
typedef __attribute__((address_space(1))) const float4 gf4_t;

REALM_DEV floatx4 mfma(half8_t a, half8_t b, floatx4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

REALM_DEV float load_x(const void *x, int bf16, size_t i)
{
    if (bf16)
        return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t *>(x)[i] << 16);
    return reinterpret_cast<const float *>(x)[i];
}

} // namespace realm_mfma

using namespace realm_mfma;

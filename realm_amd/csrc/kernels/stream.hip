// XOR checksum of a device buffer: a plain streaming read (no counterpart in
// the reference).  Workgroup b folds its contiguous share of the buffer,
// 16 bytes per lane and four loads per lane in flight, and writes one
// partial word; the checksum is the XOR of the partials.  Besides checking
// uploaded data, it measures the practical HBM read ceiling for a launch of
// a given size (nothing but the loads the data needs).
#include "common.h"

template <typename I>
REALM_DEV void checksum_body(const uint8_t *__restrict__ buf, long long nbytes,
                             uint32_t *__restrict__ partials)
{
    __shared__ uint32_t red[16];
    const I n16 = (I)(nbytes >> 4);
    const I per = (n16 + gridDim.x - 1) / gridDim.x;
    const I s = (I)blockIdx.x * per, e = min(n16, s + per);
    const uint4 *p = reinterpret_cast<const uint4 *>(buf);
    uint32_t acc = 0;
    for (I i = s + threadIdx.x; i < e; i += 4096) {
        uint4 v[4];
#pragma unroll
        for (int d = 0; d < 4; ++d)
            v[d] = i + d * 1024 < e ? p[i + d * 1024] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int d = 0; d < 4; ++d)
            acc ^= v[d].x ^ v[d].y ^ v[d].z ^ v[d].w;
    }
    // the bytes past the last whole 16 (workgroup 0), as a little-endian word stream
    if (blockIdx.x == 0 && threadIdx.x < (nbytes & 15))
        acc ^= (uint32_t)buf[((size_t)n16 << 4) + threadIdx.x] << (8 * (threadIdx.x & 3));
    for (int off = 32; off > 0; off >>= 1)
        acc ^= __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t r = 0;
        for (int w = 0; w < 16; ++w)
            r ^= red[w];
        partials[blockIdx.x] = r;
    }
}

// 32-bit positions below 2^31 sixteen-byte chunks (32 GB), 64-bit beyond
extern "C" __global__ __launch_bounds__(1024) void realm_checksum(const uint8_t *__restrict__ buf,
                                                                  long long nbytes,
                                                                  uint32_t *__restrict__ partials)
{
    if ((nbytes >> 4) < (1LL << 31))
        checksum_body<uint32_t>(buf, nbytes, partials);
    else
        checksum_body<unsigned long long>(buf, nbytes, partials);
}

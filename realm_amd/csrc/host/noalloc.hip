// The fixed scratch region of the library's no-allocation entry point
// (realm_hip_weights_matmul_noalloc_dev): a file-scope device array, so that
// callers who cannot allocate (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc) still get the activation staging
// and K-split partials the batched products need.  Each GPU holds its own
// copy of the array, at its own address, until the process ends.
//
// Compiled by hipcc (host + gfx950 device code) into an object of the host
// library; the HIP runtime registers the array at library load.  In host
// code the array's name is only a stand-in: its device address comes from
// hipGetSymbolAddress, taken once per device with that device current.
#include <hip/hip_runtime.h>

#include "noalloc.h"

static __device__ __align__(256) unsigned char scratch[REALM_NOALLOC_SCRATCH_BYTES];

extern "C" int realm_noalloc_scratch_address(void **ptr)
{
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
        *ptr = nullptr;
        return (int)(e == hipSuccess ? hipErrorInvalidSymbol : e);
    }
    *ptr = p;
    return 0;
}

// Size of the no-allocation entry point's fixed scratch region, and the call
// (noalloc.hip) that returns the current device's copy of it.
#pragma once

#define REALM_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

#ifdef __cplusplus
extern "C" {
#endif

// Device address of the scratch array on the current device (0, or a
// hipError_t value with *ptr = NULL).
int realm_noalloc_scratch_address(void **ptr);

#ifdef __cplusplus
}
#endif

// Translation unit of the GEMV variants of one weight format, selected with
// -DREALM_GEMV_FMT=0 (Q4_K), 1 (Q6_K), 2 (Q8_0) or 3 (the 32-element formats in
// the q8m layout), and one token count,
// -DREALM_GEMV_NT=1 (default), 2 or 4; or, with -DREALM_GEMV_PRE, the
// decoder layer's one-token kernels with the RMSNorm or SwiGLU fused in.
#ifndef REALM_GEMV_FMT
#error "REALM_GEMV_FMT must be defined"
#endif
#include "gemv.hip"

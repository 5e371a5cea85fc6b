// Kernel-argument structs shared by the host library (g++) and the gfx950
// kernels (hipcc): plain C layouts, passed by value through
// hipModuleLaunchKernel.
#pragma once

#include <stdint.h>

#ifdef __cplusplus
namespace realm {
#endif

// One registered LoRA adapter, as the kernels read it from the device table.
struct LoraEntry {
    const void *a; // [rank][in_dim], f32 or f16
    const void *b; // [out_dim][rank], f32 or f16
    int32_t rank;
    int32_t dtype; // 0 f32, 1 f16
    float scale;   // alpha / rank
    int32_t pad;
};

// One 16-row chunk of one adapter's A (the fused shrink's unit of work):
// the set lists the chunks that exist (rc * 16 < rank), with their entry.
struct LoraChunk {
    LoraEntry e;
    int32_t a;  // adapter slot
    int32_t rc; // rows 16 rc .. 16 rc + 15
    int32_t pad[2];
};

#define REALM_GEMM_MAX_SEGS 4

// Arguments of the LoRA shrink and expand kernels: one launch covers up to
// REALM_GEMM_MAX_SEGS projections that share the input and the token ids
// (e.g. q and v), each with its own adapter set.  The adapter slots of the
// projections are concatenated along grid x: projection p owns slots
// a_start[p] .. a_start[p + 1] - 1 (unused entries hold INT32_MAX).
struct LoraGroupArgs {
    const void *xh;            // shrink: prepared activations (f16 hi)
    const void *xl;            // shrink: f16 lo part (null for bf16 input)
    const float *tscale;       // shrink: per-token scales (NaN: exact path)
    const void *x;             // shrink: the caller's activations [M][K] (exact path)
    const int32_t *ids;        // adapter slot per token (-1 none)
    int32_t xbf16;             // x is bf16 (else f32)
    int32_t M, K, KX;
    int32_t nparts;            // shrink K parts (512 positions each; fused: LORA_FUSED_KP)
    int32_t a_start[REALM_GEMM_MAX_SEGS + 1];
    // fused shrink (workgroups of the xprep launch past its token rows):
    // projection p owns shrink workgroups wg_start[p] .. wg_start[p + 1] - 1,
    // one per (entry of its set's chunk list, K part)
    int32_t wg_start[REALM_GEMM_MAX_SEGS + 1];
    const LoraChunk *chunks[REALM_GEMM_MAX_SEGS];
    const LoraEntry *table[REALM_GEMM_MAX_SEGS];
    float *u[REALM_GEMM_MAX_SEGS];        // shrink output [part][token][rmax]
    float *y[REALM_GEMM_MAX_SEGS];        // expand: outputs [M][N] (hold the base product)
    int32_t N[REALM_GEMM_MAX_SEGS];
    int32_t rmax[REALM_GEMM_MAX_SEGS];    // largest rank of the set, rounded up to 8
    int32_t pstride[REALM_GEMM_MAX_SEGS]; // floats per part of u
};

// K positions per part of the fused shrink (the expand, folded into the
// K-split reduce, adds the parts in order); ranks up to LORA_FUSED_RMAX.
#define LORA_FUSED_KP 2048
#define LORA_FUSED_RMAX 128
#define LORA_FUSED_MAX_M 64 // tokens per call

// Arguments of the realm_gemm_* kernels.
struct GemmArgs {
    const void *w0;     // Q4_K hdr | Q6_K d  | Q8_0 d
    const void *w1;     // Q4_K qs  | Q6_K sc | Q8_0 q
    const void *w2;     // Q6_K q
    const void *xh;     // f16 activations, hi part [Mp][KX]
    const void *xl;     // f16 lo part (null for bf16 input)
    const void *xm;     // Q4_K min fragments [Mp][K/256][4][8] f16
    const float *tscale; // per token 2^e; NaN: the token takes the exact path (exact.h)
    const void *x;      // the activations as the caller passed them [M][K] (exact path)
    int32_t xbf16;      // x is bf16 (else f32)
    int32_t fmt;        // 0 Q4_K, 1 Q6_K, 2 Q8_0 (the K-split reduce's exact path)
    float *y;           // [M][N]
    int32_t N, K, KX, M;
    int32_t nan_fb;
    int32_t n_adapters;
    const int32_t *ids;           // LoRA: adapter slot per token (-1 none)
    const LoraEntry *table;       // LoRA: device table
    const float *u;               // LoRA: shrink output [Mp][rmax]
    int32_t rmax;
    int32_t ksplit;               // tiled kernels: K splits (1 = none)
    float *part;                  // tiled kernels, ksplit > 1: parts, tile-major
                                  // [tile][ksplit][token in tile][row in tile]
    int32_t xt;                   // tiled kernels: XCDs along the token tiles (1, 2, 4, 8)
    // tiled kernels: the matrices of one launch (up to 4 sharing the input,
    // e.g. Q/K/V), each padded to whole row tiles; segment i owns row tiles
    // seg_tile[i] .. seg_tile[i + 1] - 1 (unused entries hold INT32_MAX)
    int32_t nseg;
    int32_t rtiles;               // row tiles of all segments
    int32_t seg_tile[REALM_GEMM_MAX_SEGS + 1];
    int32_t seg_n[REALM_GEMM_MAX_SEGS];
    const void *seg_w0[REALM_GEMM_MAX_SEGS];
    const void *seg_w1[REALM_GEMM_MAX_SEGS];
    const void *seg_w2[REALM_GEMM_MAX_SEGS];
    float *seg_y[REALM_GEMM_MAX_SEGS];
};

// Arguments of the realm_gemv_* kernels: up to 4 matrices of one format
// that share the input x (a grouped launch, e.g. Q/K/V), rows concatenated.
#define REALM_GEMV_MAX_MATS 4
struct GemvArgs {
    const void *w0[REALM_GEMV_MAX_MATS];
    const void *w1[REALM_GEMV_MAX_MATS];
    const void *w2[REALM_GEMV_MAX_MATS];
    float *y[REALM_GEMV_MAX_MATS];
    int32_t row_start[REALM_GEMV_MAX_MATS + 1]; // prefix sums of row counts
    int32_t nmat;
    const float *x;
    int32_t K, KX;
    int32_t nan_fb;
    int32_t m; // tokens (rows of x and of each y); 1 for the one-token kernels
    // The decoder layer's step before the product, fused into the x staging
    // of the one-token "_n" and "_s" kernels (unused by the others):
    //   _n: x' = RMSNorm(x + pre_a) * pre_w (pre_a may be null), with
    //       x + pre_a written to pre_sum by workgroup 0 when pre_sum is set;
    //   _s: x' = SwiGLU(gate = x, up = pre_a).
    const float *pre_a;
    const float *pre_w;
    float *pre_sum;
    float pre_eps;
};

#ifdef __cplusplus
} // namespace realm
#endif

/*
 * realm_oracle.h -- CPU restatement of Realm's quantized compute path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP
 * implementation is compared against.  Only tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py may load it; the product library
 * (realm_amd/) never links, loads or calls it.
 *
 * Every function restates one reference function; the citation is given at
 * the definition in realm_oracle.c.  The reference is a Rust workspace that
 * cannot be compiled in this image (no cargo/rustc), so there is no build of
 * the reference itself to check against; the restatement is pinned instead by
 * the reference's own known-answer tests, closed forms and fp64 brute force
 * (see tests/test_oracle.py).
 *
 * Status codes follow realm-runtime's C-ABI ErrorCode
 * (crates/realm-runtime/src/lib.rs:110-135):
 *   0 Ok, 1 GenericFailure, 3 InvalidArgument (Error::InvalidShape),
 *   4 ModelParseError (Error::InvalidFormat).
 * RO_PANIC (-1) marks inputs on which the reference panics (slice out of
 * range) instead of returning an error.
 */
#ifndef REALM_ORACLE_H
#define REALM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RO_OK 0
#define RO_GENERIC_FAILURE 1
#define RO_INVALID_ARGUMENT 3
#define RO_MODEL_PARSE_ERROR 4
#define RO_PANIC (-1)

/* ggml type ids (crates/realm-core/src/formats/gguf.rs:458-480) */
#define RO_GGML_Q4_0 2
#define RO_GGML_Q4_1 3
#define RO_GGML_Q5_0 6
#define RO_GGML_Q5_1 7
#define RO_GGML_Q8_0 8
#define RO_GGML_Q8_1 9
#define RO_GGML_Q2_K 10
#define RO_GGML_Q3_K 11
#define RO_GGML_Q4_K 12
#define RO_GGML_Q5_K 13
#define RO_GGML_Q6_K 14
#define RO_GGML_Q8_K 15

#define RO_QK_K 256
#define RO_QK8_0 32

/* Block layouts, byte-identical to the #[repr(C)] structs of
 * crates/realm-core/src/quant.rs (Q8_0 :52-59, Q4_K :97-107, Q6_K :191-198). */
typedef struct {
    uint16_t d;
    uint16_t dmin;
    uint8_t scales[12];
    uint8_t qs[128];
} ro_block_q4_k; /* 144 bytes */

typedef struct {
    uint8_t ql[128];
    uint8_t qh[64];
    int8_t scales[16];
    uint16_t d;
} ro_block_q6_k; /* 210 bytes */

typedef struct {
    uint16_t scale;
    int8_t quants[32];
} ro_block_q8_0; /* 34 bytes */

/* IEEE binary16 <-> binary32 (the `half` crate's f16::to_f32 / from_f32). */
float ro_f16_to_f32(uint16_t h);
/* Bytes per block of the 32-element formats Q4_0/Q4_1/Q5_0/Q5_1/Q8_1 (0 for
 * others). */
int ro_block32_bytes(int type);
/* bytes of one 256-element block of the reference's own Q2_K / Q3_K / Q5_K /
 * Q8_K layouts (their #[repr(C)] sizes), 0 for other types */
int ro_kquant_bytes(int type);
uint16_t ro_f32_to_f16(float f);

void ro_get_scale_min_k4(int j, const uint8_t *scales, uint8_t *sc, uint8_t *m);

int ro_dequantize_q4_k(const ro_block_q4_k *b, float *out256);
int ro_dequantize_q6_k(const ro_block_q6_k *b, float *out256);
int ro_dequantize_q8_0(const ro_block_q8_0 *b, float *out32);
int ro_dequantize_tensor(const uint8_t *data, size_t nbytes, int ggml_type,
                         size_t element_count, float *out);

/* fused.rs semantics (portable scalar order, no FMA contraction). */
int ro_fused_q4k(const ro_block_q4_k *blocks, size_t nblocks, const float *input,
                 size_t input_len, float *out, size_t batch, size_t n, size_t k,
                 int nan_fallback);
int ro_fused_q6k(const ro_block_q6_k *blocks, size_t nblocks, const float *input,
                 size_t input_len, float *out, size_t batch, size_t n, size_t k,
                 int nan_fallback);
int ro_fused_q80(const ro_block_q8_0 *blocks, size_t nblocks, const float *input,
                 size_t input_len, float *out, size_t batch, size_t n, size_t k);

/* CandleCpuBackend semantics: dequantize everything, then x . W^T. */
int ro_candle_fused(int ggml_type, const void *blocks, size_t nblocks,
                    const float *input, size_t input_len, float *out,
                    size_t batch, size_t n, size_t k);

/* gemm.rs dense kernels. */
int ro_matmul_f32(const float *a, size_t a_len, const float *b, size_t b_len,
                  float *c, size_t m, size_t k, size_t n);
int ro_matmul_transposed(const float *a, size_t a_len, const float *bt,
                         size_t bt_len, float *c, size_t m, size_t k, size_t n);

/* lora.rs merge: out = W + (alpha/rank) * (B @ A). */
int ro_lora_apply_to_weights(const float *base, size_t base_len, const float *lora_a,
                             size_t a_len, const float *lora_b, size_t b_len,
                             size_t rank, float alpha, size_t out_dim, size_t in_dim,
                             float *out);

/* Unmerged multi-adapter closed form, f32 sequential sums:
 *   y[t] = base[t] + (alpha_a/r_a) * B_a (A_a x[t])   for ids[t] >= 0.
 * a_ptrs/b_ptrs are f32 row-major A [r x k], B [n x r]. */
int ro_multi_lora_delta(const float *x, size_t batch, size_t k, size_t n,
                        const int32_t *ids, size_t n_adapters,
                        const float *const *a_ptrs, const float *const *b_ptrs,
                        const int32_t *ranks, const float *alphas, float *y);

/* fp64 brute force y[b,n] = sum_k w[n,k] x[b,k]  (w already dequantized). */
void ro_matvec_f64(const float *w, const float *x, double *y, size_t batch,
                   size_t n, size_t k);

/* Row-parallel OpenMP variant of ro_candle_fused used only as the CPU
 * baseline timing (dequantize row, then dot).  Returns the thread count. */
int ro_fused_parallel(int ggml_type, const void *blocks, const float *input,
                      float *out, size_t batch, size_t n, size_t k, int threads);

#ifdef __cplusplus
}
#endif
#endif

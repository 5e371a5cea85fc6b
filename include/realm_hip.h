/*
 * realm_hip.h -- C ABI of the MI355X (gfx950) quantized compute path.
 *
 * This is the drop-in boundary for Realm's quantized dequant x matmul path.
 * The Rust host binds it with `extern "C"` behind its
 * existing GpuBackendTrait and candle_matmul host functions.  All pointers are
 * plain C pointers; sizes are element counts unless named *_bytes / nbytes.
 *
 * Conventions (all entry points):
 *  - Return a realm_status (0 = Ok).  On failure a message is stored in a
 *    thread-local slot read with realm_hip_last_error(), as the reference's
 *    C ABI does (crates/realm-runtime/src/lib.rs:137-150).
 *  - Inputs are borrowed for the duration of the call; outputs are allocated
 *    by the caller.  Host-pointer entry points are synchronous.
 *  - Weight layout on the host is the reference's: N rows of K/QK packed
 *    blocks, row-major by output feature (crates/realm-compute-cpu/src/
 *    fused.rs:266), blocks byte-identical to crates/realm-core/src/quant.rs
 *    (Q8_0 34 B :52-59, Q4_K 144 B :97-107, Q6_K 210 B :191-198).
 *  - Matmul semantics: out[b*n + j] = sum_k W[j,k] * input[b*k + k]
 *    (x . W^T), f32 output.
 *  - Any thread may call; each thread gets its own HIP stream.  The weight
 *    and adapter registries are guarded by a mutex.
 */
#ifndef REALM_HIP_H
#define REALM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define REALM_HIP_ABI_VERSION 2

/* Error codes: crates/realm-runtime/src/lib.rs:110-135 (ErrorCode) and the
 * From<realm_core::Error> mapping there: InvalidShape -> InvalidArgument,
 * BackendError -> BackendUnsupported, Runtime -> GenericFailure. */
typedef enum realm_status {
    REALM_OK = 0,
    REALM_GENERIC_FAILURE = 1,
    REALM_OUT_OF_MEMORY = 2,
    REALM_INVALID_ARGUMENT = 3,
    REALM_MODEL_PARSE_ERROR = 4,
    REALM_BACKEND_UNSUPPORTED = 5,
    REALM_SHADER_COMPILE_ERROR = 6,
    REALM_IO_ERROR = 7
} realm_status;

/* ggml tensor type ids (crates/realm-core/src/formats/gguf.rs:458-480). */
#define REALM_GGML_F32 0
#define REALM_GGML_Q4_0 2
#define REALM_GGML_Q4_1 3
#define REALM_GGML_Q5_0 6
#define REALM_GGML_Q5_1 7
#define REALM_GGML_Q8_0 8
#define REALM_GGML_Q8_1 9
#define REALM_GGML_Q2_K 10
#define REALM_GGML_Q3_K 11
#define REALM_GGML_Q4_K 12
#define REALM_GGML_Q5_K 13
#define REALM_GGML_Q6_K 14
#define REALM_GGML_Q8_K 15

/* Adapter storage dtypes for LoRA A/B. */
#define REALM_DTYPE_F32 0
#define REALM_DTYPE_F16 1

/* ------------------------------------------------------------ lifecycle */

/* Select the device, load the gfx950 code object (hipModuleLoadData) and
 * resolve every kernel.  Idempotent; other entry points call it lazily on
 * device 0.  Replaces backend construction in Memory64Runtime::
 * create_gpu_backend (crates/realm-runtime/src/memory64_host.rs:446-465). */
int realm_hip_init(int device);

/* Thread-local message of the last failed call on this thread ("" if none).
 * crates/realm-runtime/src/lib.rs:137-150 (set_last_error/take_last_error). */
const char *realm_hip_last_error(void);

/* Name of the last kernel this thread launched through the library ("" if
 * none): a diagnostic for profilers and benchmarks, so that a timing can be
 * matched to the kernel variant the dispatcher chose.  No counterpart in the
 * reference (its backends have no kernel variants). */
const char *realm_hip_last_kernel(void);

/* GpuBackendTrait::name (crates/realm-compute-gpu/src/gpu_backend_trait.rs:142). */
const char *realm_hip_backend_name(void);

/* fused.rs replaces NaN/Inf super-block scales by constants
 * (crates/realm-compute-cpu/src/fused.rs:276-285, 1171-1175); quant.rs and
 * the Candle backends do not.  0 (default) = quant.rs behaviour, 1 = fused.rs
 * behaviour.  Process-wide. */
int realm_hip_set_nan_fallback(int enable);

/* ------------------------------------------- GpuBackendTrait (host slices) */

/* GpuBackendTrait::matmul (gpu_backend_trait.rs:18-20): C = A @ B with A
 * [m,k], B [k,n] row-major f32; out has m*n elements. */
int realm_hip_matmul(const float *a, size_t a_len, const float *b, size_t b_len,
                     uint32_t m, uint32_t k, uint32_t n, float *out);

/* The same product on device pointers, asynchronous on `stream` (NULL = this
 * thread's stream), for callers whose operands already live on the device:
 * C [m,n] = A [m,k] @ B, B [k,n] row-major, or B^T with B [n,k] when
 * b_transposed is non-zero (candle_matmul_transposed,
 * memory64_host.rs:971-1086).  f32 products and sums on MFMA. */
int realm_hip_matmul_dev(const float *d_a, const float *d_b, float *d_c, uint32_t m,
                         uint32_t k, uint32_t n, int b_transposed, void *stream);

/* GpuBackendTrait::fused_dequant_matmul_q4k / _q6k / _q80
 * (gpu_backend_trait.rs:22-29, 42-49, 122-129).  Validation as in the
 * reference backends (crates/realm-compute-gpu/src/candle_backend.rs:448-464,
 * 1115-1131; lib.rs:339-345): k % 256 == 0 (k % 32 == 0 for Q8_0), n_blocks
 * == n*k/QK and input_len == batch_size*k, else REALM_INVALID_ARGUMENT.
 * out has batch_size*n elements.  Weights are uploaded for this call only;
 * use realm_hip_weights_register for device-resident weights. */
int realm_hip_fused_dequant_matmul_q4k(const void *blocks, size_t n_blocks,
                                       const float *input, size_t input_len,
                                       size_t batch_size, size_t n, size_t k,
                                       float *out);
int realm_hip_fused_dequant_matmul_q6k(const void *blocks, size_t n_blocks,
                                       const float *input, size_t input_len,
                                       size_t batch_size, size_t n, size_t k,
                                       float *out);
int realm_hip_fused_dequant_matmul_q80(const void *blocks, size_t n_blocks,
                                       const float *input, size_t input_len,
                                       size_t batch_size, size_t n, size_t k,
                                       float *out);

/* GpuBackendTrait::fused_dequant_matmul_q40 / _q41 / _q50 / _q51 / _q81
 * (gpu_backend_trait.rs:82-119, 132-139) on the reference's 32-element block
 * layouts (crates/realm-core/src/quant.rs:10-70: Q4_0 18 B, Q4_1 20 B, Q5_0
 * 22 B, Q5_1 24 B, Q8_1 36 B per block), as CandleGpuBackend computes them
 * (candle_backend.rs:837-1103): validation k % 32 == 0, n_blocks == n*k/32,
 * input_len == batch_size*k; the blocks dequantized bit-exactly on the
 * device (quant.rs:226-370), then y = x W^T on the f32 MFMA GEMM. */
int realm_hip_fused_dequant_matmul_q40(const void *blocks, size_t n_blocks,
                                       const float *input, size_t input_len,
                                       size_t batch_size, size_t n, size_t k, float *out);
int realm_hip_fused_dequant_matmul_q41(const void *blocks, size_t n_blocks,
                                       const float *input, size_t input_len,
                                       size_t batch_size, size_t n, size_t k, float *out);
int realm_hip_fused_dequant_matmul_q50(const void *blocks, size_t n_blocks,
                                       const float *input, size_t input_len,
                                       size_t batch_size, size_t n, size_t k, float *out);
int realm_hip_fused_dequant_matmul_q51(const void *blocks, size_t n_blocks,
                                       const float *input, size_t input_len,
                                       size_t batch_size, size_t n, size_t k, float *out);
int realm_hip_fused_dequant_matmul_q81(const void *blocks, size_t n_blocks,
                                       const float *input, size_t input_len,
                                       size_t batch_size, size_t n, size_t k, float *out);

/* GpuBackendTrait::fused_dequant_matmul_q5k / _q8k / _q2k / _q3k
 * (gpu_backend_trait.rs:31-79) on the reference's own 256-element layouts
 * (crates/realm-core/src/quant.rs:71-95, 200-222: the #[repr(C)] sizes Q5_K
 * 178 B, Q8_K 292 B, Q2_K 116 B, Q3_K 196 B, which are not ggml's), as
 * CandleGpuBackend computes them (candle_backend.rs:507-571, 639-836):
 * k % 256 == 0 and n_blocks == n*k/256 (else REALM_INVALID_ARGUMENT), an
 * input of another length fails as the reference's tensor creation does
 * (REALM_GENERIC_FAILURE); the blocks are dequantized bit-exactly on the
 * device (quant.rs:453-638, including Q5_K's zero upper half), then
 * y = x W^T on the f32 MFMA GEMM.  Registered as resident weights they stay
 * dequantized (f32), like the 32-element formats. */
int realm_hip_fused_dequant_matmul_q5k(const void *blocks, size_t n_blocks,
                                       const float *input, size_t input_len,
                                       size_t batch_size, size_t n, size_t k, float *out);
int realm_hip_fused_dequant_matmul_q8k(const void *blocks, size_t n_blocks,
                                       const float *input, size_t input_len,
                                       size_t batch_size, size_t n, size_t k, float *out);
int realm_hip_fused_dequant_matmul_q2k(const void *blocks, size_t n_blocks,
                                       const float *input, size_t input_len,
                                       size_t batch_size, size_t n, size_t k, float *out);
int realm_hip_fused_dequant_matmul_q3k(const void *blocks, size_t n_blocks,
                                       const float *input, size_t input_len,
                                       size_t batch_size, size_t n, size_t k, float *out);

/* Format-generic form of the eight above (ggml_type 2, 3, 6, 7, 8, 9, 12 or
 * 14).  The trait's Q2_K, Q3_K, Q5_K and Q8_K forms return
 * REALM_BACKEND_UNSUPPORTED so that dispatch_matmul falls back to the CPU
 * (crates/realm-models/src/matmul_dispatch.rs:72-88). */
int realm_hip_fused_dequant_matmul(int ggml_type, const void *blocks, size_t n_blocks,
                                   const float *input, size_t input_len,
                                   size_t batch_size, size_t n, size_t k, float *out);

/* ----------------------------------------- candle_matmul host functions */

/* env.candle_matmul / env.candle_matmul_transposed
 * (crates/realm-runtime/src/memory64_host.rs:853-969, 971-1086) over a
 * tenant's linear memory `mem` of mem_len bytes.  A [m,k] at a_ptr, B [k,n]
 * (or [n,k] when transposed) at b_ptr, C [m,n] written at result_ptr, all
 * little-endian f32.  Returns m*n on success, -3 when A is out of bounds, -4
 * when B is, -5 on a compute failure, -6 when C does not fit (the reference's
 * -2 "no memory export" has no counterpart: the caller passes the memory). */
int32_t realm_hip_candle_matmul(uint8_t *mem, size_t mem_len, uint32_t a_ptr,
                                uint32_t b_ptr, uint32_t result_ptr, uint32_t m,
                                uint32_t k, uint32_t n);
int32_t realm_hip_candle_matmul_transposed(uint8_t *mem, size_t mem_len, uint32_t a_ptr,
                                           uint32_t b_ptr, uint32_t result_ptr,
                                           uint32_t m, uint32_t k, uint32_t n);

/* --------------------------------------------------------- dequantize */

/* dequantize_tensor (crates/realm-core/src/quant.rs:663-770) on the GPU,
 * bit-exact with dequantize_q4_k / _q6_k / _q8_0 (quant.rs:127-187, 393-451,
 * 371-387).  Q4_K: nbytes % 144 != 0 -> REALM_MODEL_PARSE_ERROR, element
 * count mismatch -> REALM_INVALID_ARGUMENT.  Q6_K / Q8_0 ignore a trailing
 * partial block and zero-fill elements past the last block; an
 * element_count smaller than the blocks' output (a panic in the reference)
 * is REALM_INVALID_ARGUMENT. */
int realm_hip_dequantize(int ggml_type, const void *data, size_t nbytes,
                         size_t element_count, float *out);

/* -------------------------------------------- device-resident weights */

/* Upload a [n,k] quantized matrix once and keep it in HBM in the device
 * layout (repacked on the GPU).  Replaces the per-call f32 upload of
 * CandleGpuBackend (candle_backend.rs:484-490) for the weights that
 * realm_forward_layer reads every call (memory64_host.rs:1958-2225).
 * ggml_type is 12 (Q4_K), 14 (Q6_K) or 8 (Q8_0); the 32-element formats 2
 * (Q4_0), 3 (Q4_1), 6 (Q5_0), 7 (Q5_1) and 9 (Q8_1) are kept dequantized
 * (f32, 4 bytes per weight) and multiply on the f32 GEMM; they take no bf16
 * input and no LoRA (REALM_BACKEND_UNSUPPORTED). */
int realm_hip_weights_register(int ggml_type, const void *blocks, size_t nbytes,
                               size_t n, size_t k, uint64_t *handle);
int realm_hip_weights_release(uint64_t handle);
int realm_hip_weights_info(uint64_t handle, int *ggml_type, size_t *n, size_t *k,
                           size_t *device_bytes);

/* y = x . W^T with resident W; host x [batch,k] f32 in, host y [batch,n] out. */
int realm_hip_weights_matmul(uint64_t handle, const float *input, size_t batch,
                             float *out);

/* Same with device pointers on a caller stream (NULL = this thread's stream);
 * asynchronous.  x is f32 [batch,k]; y is f32 [batch,n]. */
int realm_hip_weights_matmul_dev(uint64_t handle, const float *d_input, size_t batch,
                                 float *d_out, void *stream);

/* No counterpart in the reference: for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  realm_hip_weights_matmul_dev's product, but every scratch
 * buffer (activation staging, K-split partials) is cut from a fixed 32 MiB
 * device array the library holds per GPU until the process ends, so the call
 * makes no hipMalloc, hipFree or other allocating call.  Needs a prior
 * realm_hip_init and an explicit stream.  A product whose staging does not
 * fit (batch x K beyond about 1,900 x 4096 for f32 input) returns
 * REALM_INVALID_ARGUMENT; K splits are reduced until their partials fit.
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (several streams or threads at once) race. */
int realm_hip_weights_matmul_noalloc_dev(uint64_t handle, const float *d_input, size_t batch,
                                         float *d_out, void *stream);

/* Grouped form for 1..4 resident weights of one format and K that share the
 * input, e.g. the q/k/v projections (or gate/up) that realm_forward_layer
 * issues back to back on the same normed hidden state
 * (crates/realm-runtime/src/memory64_host.rs:2078-2308, 2384-2443):
 * d_outs[i] = x . W_i^T.  Batches of 1-4 tokens run all of them in one
 * integer-dot GEMV launch, larger Q4_K / Q6_K batches in one tiled MFMA
 * launch. */
int realm_hip_weights_matmul_group_dev(const uint64_t *handles, size_t count,
                                       const float *d_input, size_t batch,
                                       float *const *d_outs, void *stream);

/* Prefill form with bf16 activations (raw bf16 bits, [batch,k]). */
int realm_hip_weights_matmul_bf16_dev(uint64_t handle, const uint16_t *d_input,
                                      size_t batch, float *d_out, void *stream);

/* ----------------------------------------------------------- multi-LoRA */

/* Register one adapter's factors for one projection: A [rank, in_dim] and
 * B [out_dim, rank] row-major (the LoRAWeights lora_a / lora_b of
 * crates/realm-runtime/src/lora.rs:10-23), scale alpha/rank (lora.rs:49-52).
 * dtype is REALM_DTYPE_F32 or REALM_DTYPE_F16 (raw binary16 bits); the
 * device keeps the given dtype.  rank must be 1..256. */
int realm_hip_lora_register(int dtype, const void *lora_a, const void *lora_b,
                            size_t rank, float alpha, size_t in_dim, size_t out_dim,
                            uint64_t *handle);
int realm_hip_lora_release(uint64_t handle);

/* Group adapters into a device-resident table; slot i of the set is
 * lora_handles[i].  All adapters of a set share in_dim, out_dim and dtype. */
int realm_hip_lora_set_create(const uint64_t *lora_handles, size_t count,
                              uint64_t *set_handle);
int realm_hip_lora_set_release(uint64_t set_handle);

/* Multi-tenant matmul: for every token t
 *   y[t] = W x[t] + (alpha_a/r_a) * B_a (A_a x[t])   with a = adapter_ids[t]
 * and y[t] = W x[t] when adapter_ids[t] < 0 (no adapter).  Equal, up to f32
 * rounding, to the reference's merged form W + scale*(B@A)
 * (crates/realm-runtime/src/lora.rs:91-144) applied per tenant.  Host
 * pointers, synchronous. */
int realm_hip_multi_lora_matmul(uint64_t weight_handle, uint64_t set_handle,
                                const float *input, size_t batch,
                                const int32_t *adapter_ids, float *out);

/* Device-pointer form, asynchronous on `stream` (NULL = this thread's). */
int realm_hip_multi_lora_matmul_dev(uint64_t weight_handle, uint64_t set_handle,
                                    const float *d_input, size_t batch,
                                    const int32_t *d_adapter_ids, float *d_out,
                                    void *stream);

/* Grouped form for 1..4 projections of one format and K that share the input
 * and the token adapter ids (q/k/v of realm_forward_layer,
 * crates/realm-runtime/src/memory64_host.rs:2078-2308, with LoRA applied per
 * projection as at :625-680): d_outs[i] = multi-LoRA matmul of weight i with
 * adapter set i.  The input is prepared once; the base products run as
 * one launch, the shrinks of all projections as one and their expands as
 * one.  Device pointers, asynchronous on `stream`. */
int realm_hip_multi_lora_matmul_group_dev(const uint64_t *weight_handles,
                                          const uint64_t *set_handles, size_t count,
                                          const float *d_input, size_t batch,
                                          const int32_t *d_adapter_ids,
                                          float *const *d_outs, void *stream);

/* ------------------------------------------- element-wise layer operations */

/* RMSNorm of `rows` rows of `hidden` f32 values on the device, as
 * CandleNeuralOpsBackend::rms_norm (crates/realm-compute-cpu/src/
 * candle_neural_ops_backend.rs:32-60; candle-nn ops::rms_norm:
 * y = x / sqrt(mean(x^2) + eps) * weight) where realm_forward_layer norms
 * the hidden state (crates/realm-runtime/src/memory64_host.rs:2069, 2337).
 * With d_residual set, the row is first x + residual (the residual add of
 * memory64_host.rs:2318-2324), written to d_sum when that is not NULL: the
 * add and the norm in one pass.  hidden must be a multiple of 4, every
 * pointer 16-byte aligned; d_sum may not be d_x or d_residual (d_out may be
 * d_x).  Asynchronous on `stream`. */
int realm_hip_rms_norm_dev(const float *d_x, const float *d_residual, const float *d_weight,
                           float eps, size_t rows, size_t hidden, float *d_sum, float *d_out,
                           void *stream);

/* SwiGLU of realm_forward_layer (memory64_host.rs:2419-2425):
 * out[i] = (gate[i] * (1 / (1 + exp(-gate[i])))) * up[i].  n a multiple of
 * 4, pointers 16-byte aligned; d_out may be d_gate or d_up. */
int realm_hip_swiglu_dev(const float *d_gate, const float *d_up, size_t n, float *d_out,
                         void *stream);

/* RoPE in place on x [seq_len, num_heads, head_dim] (MultiHeadAttention::
 * apply_rope, crates/realm-models/src/attention.rs:171-235): interleaved
 * pairs (i, i+1), freq = 1 / theta^(i / head_dim), angle = (start_pos + s)
 * freq.  head_dim even, x 8-byte aligned. */
int realm_hip_rope_dev(float *d_x, size_t seq_len, size_t num_heads, size_t head_dim,
                       size_t start_pos, float theta, void *stream);

/* Causal attention of seq_len query tokens at absolute positions position..
 * over kv_len cached tokens (MultiHeadAttention::compute_attention,
 * attention.rs:300-380, with StandardAttention,
 * crates/realm-runtime/src/attention/standard.rs:36-210): q and out are
 * [seq_len, num_heads, head_dim], the caches [kv_len, num_kv_heads,
 * head_dim] (the KVCache layout, crates/realm-models/src/kv_cache.rs:44-70);
 * query t sees keys j <= position + t, head h reads KV head
 * h / (num_heads / num_kv_heads) (repeat_kv, attention.rs:272-296), scale
 * 1/sqrt(head_dim).  head_dim divides 256; kv_len beyond what one
 * workgroup's LDS holds for the scores -> REALM_BACKEND_UNSUPPORTED. */
int realm_hip_attention_dev(const float *d_q, const float *d_k_cache, const float *d_v_cache,
                            size_t seq_len, size_t kv_len, size_t position, size_t num_heads,
                            size_t num_kv_heads, size_t head_dim, float *d_out, void *stream);

/* KVCache::append (kv_cache.rs:44-70): copy seq_len rows of kv_dim keys and
 * values into the device caches after the cur_len cached rows; more than
 * max_len rows -> REALM_MODEL_PARSE_ERROR ("KV cache overflow", as the
 * reference's Error::ParseError). */
int realm_hip_kv_append_dev(const float *d_k, const float *d_v, size_t seq_len, size_t kv_dim,
                            size_t cur_len, size_t max_len, float *d_k_cache, float *d_v_cache,
                            void *stream);

/* Residual add out = a + b (CandleCpuBackend::add where realm_forward_layer
 * adds the attention and FFN outputs, memory64_host.rs:2318-2324,
 * 2452-2458).  n a multiple of 4, pointers 16-byte aligned. */
int realm_hip_add_dev(const float *d_a, const float *d_b, size_t n, float *d_out, void *stream);

/* One decoder layer's weights and shape for realm_hip_forward_layer_dev:
 * registered weight handles (Wq, Wo [hidden x hidden], Wk, Wv [kv_heads *
 * head_dim x hidden], W_gate, W_up [intermediate x hidden], W_down
 * [hidden x intermediate]), the two norm weight vectors on the device, and
 * the TransformerConfig fields the layer reads (gguf.rs:212-280).
 *
 * Per-tenant LoRA (apply_lora_to_weight_format on each of the seven
 * projections, memory64_host.rs:625-680, 2232-2274, 2347-2378, with keys
 * layer.N.attn_q .. ffn_down as lora_integration.rs:198-270 builds them):
 * lora_q .. lora_down are adapter sets (realm_hip_lora_set_create, 0 = no
 * adapters on that projection) whose slot t holds tenant t's adapter for it;
 * token i of the call uses slot d_adapter_ids[i] of every set (-1, or a slot
 * past a set's size: that projection's base product).  The reference merges
 * one tenant's delta into the weights; here y = W x + s B (A x) per token,
 * the same product, for a batch that mixes tenants.  Calls with adapters
 * take at most 1024 tokens. */
typedef struct realm_layer {
    uint64_t wq, wk, wv, wo, w_gate, w_up, w_down;
    const float *attn_norm, *ffn_norm;
    uint32_t hidden, num_heads, num_kv_heads, head_dim, intermediate;
    float rms_norm_eps, rope_theta;
    uint64_t lora_q, lora_k, lora_v, lora_o, lora_gate, lora_up, lora_down;
    const int32_t *d_adapter_ids;
} realm_layer;

/* realm_forward_layer (crates/realm-runtime/src/memory64_host.rs:1915-2472)
 * on the device for seq_len tokens at absolute positions position.. :
 * RMSNorm, Q/K/V, RoPE, KV-cache append (K and V rows written at row
 * `position` of the [max_seq_len, kv_heads * head_dim] caches), causal
 * attention over the position + seq_len cached rows, Wo, residual, FFN
 * RMSNorm, gate/up, SwiGLU, W_down, residual.  d_hidden and d_out are
 * [seq_len, hidden] f32 (they may not overlap).  Asynchronous on `stream`;
 * every step is a kernel or a library product on that stream, so a decode
 * step can be captured in a HIP graph after one eager call.  Overflowing the
 * cache -> REALM_MODEL_PARSE_ERROR, as KVCache::append. */
int realm_hip_forward_layer_dev(const realm_layer *layer, const float *d_hidden, size_t seq_len,
                                size_t position, float *d_k_cache, float *d_v_cache,
                                size_t max_seq_len, float *d_out, void *stream);

/* n_layers such layers back to back (the layer loop around realm_forward_layer,
 * Model::forward, crates/realm-models/src/model.rs:598-601): layer l reads
 * d_k_caches[l] / d_v_caches[l]; between layers the residual add is fused
 * into the next layer's first RMSNorm (one launch fewer per layer), and
 * d_out receives the last layer's output.  Same contract as
 * realm_hip_forward_layer_dev otherwise. */
int realm_hip_forward_layers_dev(const realm_layer *layers, size_t n_layers,
                                 const float *d_hidden, size_t seq_len, size_t position,
                                 float *const *d_k_caches, float *const *d_v_caches,
                                 size_t max_seq_len, float *d_out, void *stream);

/* ------------------------------------------------------ GGUF model images */

/* The transformer shape a GGUF image declares: GGUFParser::extract_config
 * (crates/realm-core/src/formats/gguf.rs:212-280), with its keys
 * ("<arch>.embedding_length", then "<arch>.hidden_size", ...) and defaults. */
typedef struct realm_gguf_config {
    uint32_t vocab_size, hidden_size, num_layers, num_heads, num_kv_heads;
    uint32_t intermediate_size, max_seq_len;
    float rms_norm_eps, rope_theta;
} realm_gguf_config;

/* Parse a GGUF image held in memory (the bytes ModelStorage::store_model
 * receives, crates/realm-runtime/src/model_storage.rs:386-395): magic,
 * version 2..3, metadata key/values, tensor table (GGUFParser::parse_header,
 * gguf.rs:111-160, 300-480).  Host only: no device call.  Errors as the
 * reference's: bad magic, version or value type -> REALM_MODEL_PARSE_ERROR;
 * an image that ends inside the header -> REALM_IO_ERROR; an empty shape or
 * a zero dimension -> REALM_INVALID_ARGUMENT (Shape::validate,
 * crates/realm-core/src/tensor.rs:102-110).  The data section starts at the
 * end of the tensor table rounded up to general.alignment (32 when absent,
 * gguf.rs:165-175).  *model is a handle for the calls below. */
int realm_hip_gguf_parse(const void *bytes, size_t len, uint64_t *model);

/* Header counts and the data section's byte offset (gguf.rs:120-135, 165-175). */
int realm_hip_gguf_info(uint64_t model, uint32_t *version, uint64_t *tensor_count,
                        uint64_t *kv_count, uint64_t *data_offset);

/* Tensor `index` of the table (TensorDesc, gguf.rs:427-455): its name
 * (NUL-terminated into name[name_cap]), ggml type, number of dimensions,
 * the dimensions padded with 1 to four (ggml order: dims4[0] is the row
 * length), its absolute byte offset in the image and its byte size (F32,
 * F16, Q8_0 as 34-byte blocks, Q4_K, Q6_K; 0 for other types).  Any output
 * pointer may be NULL. */
int realm_hip_gguf_tensor(uint64_t model, size_t index, char *name, size_t name_cap,
                          int *ggml_type, uint32_t *n_dims, uint64_t *dims4,
                          uint64_t *abs_offset, uint64_t *nbytes);

/* Index of the tensor named `name` (the last one, for a repeated name, as
 * StoredModel::add_tensor keeps it, model_storage.rs:286-290, 472). */
int realm_hip_gguf_find(uint64_t model, const char *name, size_t *index);

/* Metadata lookups: MetadataValue::as_u32 (any integer type, truncated) and
 * as_string (gguf.rs:50-85). */
int realm_hip_gguf_meta_u32(uint64_t model, const char *key, uint32_t *out);
int realm_hip_gguf_meta_str(uint64_t model, const char *key, char *buf, size_t cap);

/* GGUFParser::extract_config (gguf.rs:212-280). */
int realm_hip_gguf_config(uint64_t model, realm_gguf_config *cfg);

/* Upload every 2-D Q4_K / Q6_K / Q8_0 tensor (and Q4_0 / Q4_1 / Q5_0 / Q5_1
 * / Q8_1, resident dequantized) of a parsed image once, as
 * resident device weights (realm_hip_weights_register with n = dims4[1],
 * k = dims4[0]), in place of the per-call tensor copies of
 * ModelStorage / quantized_to_weight_format (model_storage.rs:444-487,
 * crates/realm-runtime/src/memory64_host.rs:2078-2225).  `bytes` must be
 * the image that was parsed; it is read during the call only.  A tensor
 * that extends past the image -> REALM_MODEL_PARSE_ERROR.  Tensors already
 * registered are skipped; *registered (may be NULL) counts this call's. */
int realm_hip_gguf_register(uint64_t model, const void *bytes, size_t len,
                            size_t *registered);

/* The registered weight handle of tensor `name` and its shape (output rows
 * n, row length k), for realm_hip_weights_matmul* and the multi-LoRA calls.
 * A tensor that is not a registered weight -> REALM_BACKEND_UNSUPPORTED. */
int realm_hip_gguf_weight(uint64_t model, const char *name, uint64_t *weight, size_t *n,
                          size_t *k);

/* Forget a parsed image and release the device weights registered from it. */
int realm_hip_gguf_release(uint64_t model);

/* -------------------------------------------------------- HIP graphs */

/* Capture the device-pointer calls issued on `stream` (not NULL) between
 * begin and end into a replayable HIP graph, for launch-bound loops such as a
 * decode step.  Run the same calls once eagerly before capturing so that the
 * library's scratch buffers are already sized.  No memset is recorded into a
 * graph.  While a graph captured on a stream is alive, the stream's scratch
 * buffers are never freed: a later, larger eager call on that stream gets new
 * buffers and the replaced ones are kept until the stream's last graph is
 * released, so replays stay valid. */
int realm_hip_graph_begin(void *stream);
int realm_hip_graph_end(void *stream, uint64_t *graph_handle);
int realm_hip_graph_launch(uint64_t graph_handle, void *stream);
int realm_hip_graph_release(uint64_t graph_handle);

/* The scratch buffers of `stream` (NULL = this thread's): bytes held,
 * replaced buffers kept for live graphs, live graphs captured on it.  No
 * counterpart in the reference (which has no device scratch); for tests and
 * memory accounting. */
int realm_hip_workspace_info(void *stream, size_t *bytes, size_t *retired, int *graphs);

/* ------------------------------------------------------------ checksum */

/* XOR of the little-endian 32-bit words of a device buffer (a trailing
 * partial word zero-padded): an integrity check of uploaded data, read once
 * at the HBM streaming rate.  No counterpart in the reference.  The _dev
 * form launches n_partials (1..4096) workgroups on `stream`, each folding a
 * contiguous share into d_partials[i]; the checksum is the XOR of the
 * partials.  The plain form returns it, synchronously. */
int realm_hip_checksum_dev(const void *d_buf, size_t nbytes, uint32_t *d_partials,
                           size_t n_partials, void *stream);
int realm_hip_checksum(const void *d_buf, size_t nbytes, uint32_t *checksum);

/* ----------------------------------------- device memory and timing */

/* Plumbing for callers without another GPU runtime (tests, bench): device
 * buffers, copies, streams and events on this library's HIP runtime. */
int realm_hip_malloc(void **d_ptr, size_t nbytes);
int realm_hip_free(void *d_ptr);
int realm_hip_memcpy_htod(void *d_dst, const void *h_src, size_t nbytes);
int realm_hip_memcpy_dtoh(void *h_dst, const void *d_src, size_t nbytes);
int realm_hip_memcpy_dtod(void *d_dst, const void *d_src, size_t nbytes);
int realm_hip_stream(void **stream);            /* this thread's stream */
int realm_hip_stream_synchronize(void *stream); /* NULL = this thread's */
int realm_hip_device_synchronize(void);
int realm_hip_event_create(void **event);
int realm_hip_event_destroy(void *event);
int realm_hip_event_record(void *event, void *stream);
int realm_hip_event_elapsed_ms(void *start, void *stop, float *ms);

#ifdef __cplusplus
}
#endif
#endif /* REALM_HIP_H */

/*
 * mote_hip.h: C ABI of libmote_hip.so, the MI355X (gfx950) implementation of
 * Mote's Q4_0 quantized-linear path, RMSNorm and RoPE.
 *
 * Conventions (all of them those of the reference's Rust FFI,
 * crates/mote-backend-hip/src/ffi.rs:8-13): pointers are untyped device
 * pointers, streams are opaque `void*` hipStream_t handles, every launch is
 * asynchronous on the given stream, the caller owns every buffer, and the
 * return value is an `int` status where 0 means success.
 *
 * Symbols marked [reference] keep the exact signature, argument meaning and
 * status codes of the reference export they replace (file:line cited).
 * Symbols marked [new] have no counterpart in the reference.
 */
#ifndef MOTE_HIP_H
#define MOTE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- HIP runtime wrappers ------------------------------------------------ */
/* [reference] crates/mote-backend-hip/src/hipblaslt_shim.cpp:259-324, bound at
 * crates/mote-backend-hip/src/ffi.rs:42-61.  Raw hipError_t; -1 for a null
 * out-parameter.  mote_hip_stream_create also allocates the stream's 64 MiB
 * split-K scratch (so split-K linears on it allocate nothing up to that
 * size); mote_hip_stream_destroy does not wait for the stream, and frees that
 * scratch once the work queued before it has completed. */
int mote_hip_get_device_count(int* count);
int mote_hip_set_device(int ordinal);
int mote_hip_malloc(void** pointer, size_t bytes);
int mote_hip_free(void* pointer);
int mote_hip_memcpy_host_to_device(void* destination, const void* source, size_t bytes);
int mote_hip_memcpy_device_to_host(void* destination, const void* source, size_t bytes);
int mote_hip_stream_create(void** stream);
int mote_hip_stream_destroy(void* stream);
int mote_hip_stream_synchronize(void* stream);
int mote_hip_mem_get_info(size_t* free_bytes, size_t* total_bytes);

/* ---- Q4_0 quantized linear ------------------------------------------------ */
/* [reference] crates/mote-backend-hip/src/quantized_linear.hip:56-91, bound at
 * crates/mote-backend-hip/src/ffi.rs:287-326.
 * output[rows, N] (f16) = input[rows, K] (f16) x weights[N, K]^T (GGML Q4_0,
 * rows of K/32 blocks of 18 bytes), f32 accumulation, one f16 rounding.
 * Status: null pointer or K % 32 != 0 -> 1 (hipErrorInvalidValue);
 * rows == 0 or N == 0 -> 0, nothing launched; rows * N > UINT_MAX -> 9
 * (hipErrorInvalidConfiguration); K == 0 launches and writes zeros; else the
 * launch status.  K above 2^31 - 1 (64-bit sizes, as in the reference) runs
 * per-element products over K parts of each output, added in part order, with
 * the partials in the stream's split-K scratch.  Output must not alias the
 * inputs. */
int mote_hip_quantized_linear_q4_0_f16(const void* input, const void* weights, void* output,
                                       uint64_t rows, uint64_t output_features,
                                       uint64_t input_features, void* stream);

/* [new] Same as above with an f32 output [rows, N] (the reference oracle's
 * output type, crates/mote-reference/src/quantized.rs:89-144). */
int mote_hip_quantized_linear_q4_0_f32(const void* input, const void* weights, void* output,
                                       uint64_t rows, uint64_t output_features,
                                       uint64_t input_features, void* stream);

/* [new] No counterpart in the reference.  mote_hip_quantized_linear_q4_0_f32
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops or harnesses that forbid hipMalloc): the same
 * arguments, checks, statuses, plans and kernels, but the split-K partial
 * tiles (1-64 tokens where K exceeds one K slice) go to the library's static
 * 16 MiB device array instead of a per-stream buffer the library allocates;
 * nothing is allocated on any call.  Every call on one GPU shares that
 * array, and it keeps the last call's contents: calls that overlap in time on
 * one GPU (several streams or threads) race.  A problem whose partial tiles
 * need more than 16 MiB (M x N x K-parts x 4 bytes) returns 2
 * (hipErrorOutOfMemory) before any launch; K above 2^31 - 1 keeps its K-part
 * partials there too. */
int mote_hip_quantized_linear_q4_0_f32_no_alloc(const void* input, const void* weights, void* output,
                                                uint64_t rows, uint64_t output_features,
                                                uint64_t input_features, void* stream);

/* [new] Fused gate/up projection: output[rows, N] (f32) =
 * silu(input . gate^T) * (input . up^T), silu(z) = z / (1 + e^-z); gate and up
 * are Q4_0 [N, K].  up_weights == NULL means gate_weights is the concatenated
 * [2N, K] matrix with the gate rows first.  Status codes as above. */
int mote_hip_q4_0_gate_up_silu_f32(const void* input, const void* gate_weights,
                                   const void* up_weights, void* output, uint64_t rows,
                                   uint64_t output_features, uint64_t input_features,
                                   void* stream);

/* [new] Q8_0 weight-only linear, the next format of the path: the reference
 * decodes Q8_0 in its oracle (crates/mote-reference/src/quantized.rs:191-195,
 * 34-byte blocks: f16 scale + 32 int8, value v * d) but has no HIP kernel for
 * it.  Weights are raw GGML Q8_0 bytes [N, K] (2-byte aligned at least);
 * arguments, outputs and status codes as for the Q4_0 entry points above. */
int mote_hip_quantized_linear_q8_0_f16(const void* input, const void* weights, void* output,
                                       uint64_t rows, uint64_t output_features,
                                       uint64_t input_features, void* stream);
int mote_hip_quantized_linear_q8_0_f32(const void* input, const void* weights, void* output,
                                       uint64_t rows, uint64_t output_features,
                                       uint64_t input_features, void* stream);

/* [new] On-device Q4_0 decode of rows x K elements to f32, bit-identical to
 * dequantize_quantized_row (crates/mote-reference/src/quantized.rs:58-74).
 * Status: null or K % 32 != 0 -> 1; empty -> 0. */
int mote_hip_dequantize_q4_0_f32(const void* weights, void* output, uint64_t rows,
                                 uint64_t input_features, void* stream);

/* ---- K-quants: Q4_K and Q6_K (256-element super-blocks) ------------------ */
/* [new] The reference defines only their geometry
 * (crates/mote-types/src/lib.rs:39-74: Q4_K 256 elements in 144 bytes,
 * 4-byte aligned; Q6_K 256 in 210 bytes, 2-byte aligned; the GGML
 * ggml-common.h layouts) and plans their block-dot path
 * (docs/roadmap.md:26-27); it has no kernel, no FFI and no oracle for them
 * (crates/mote-reference/src/quantized.rs:154-156).  These follow the
 * Q4_0 entry points' arguments and statuses, with blocks of 256 elements:
 * null pointer, K % 256 != 0, weights below the format's alignment, an odd
 * input address or an output below its element alignment -> 1; rows == 0 or
 * N == 0 -> 0; rows * N > UINT_MAX or K > 2^31 - 1 -> 9; K == 0 writes zeros.
 * output[rows, N] = input[rows, K] (f16) x weights[N, K]^T, f32
 * accumulation, one final rounding for the f16 output. */
int mote_hip_quantized_linear_q4_k_f16(const void* input, const void* weights, void* output,
                                       uint64_t rows, uint64_t output_features,
                                       uint64_t input_features, void* stream);
int mote_hip_quantized_linear_q4_k_f32(const void* input, const void* weights, void* output,
                                       uint64_t rows, uint64_t output_features,
                                       uint64_t input_features, void* stream);
int mote_hip_quantized_linear_q6_k_f16(const void* input, const void* weights, void* output,
                                       uint64_t rows, uint64_t output_features,
                                       uint64_t input_features, void* stream);
int mote_hip_quantized_linear_q6_k_f32(const void* input, const void* weights, void* output,
                                       uint64_t rows, uint64_t output_features,
                                       uint64_t input_features, void* stream);

/* [new] On-device decode of rows x K elements to f32 (output 4-byte
 * aligned), bit-identical to GGML's dequantize_row_q4_K / dequantize_row_q6_K.
 * Status: null, K % 256 != 0 or misaligned -> 1; empty -> 0. */
int mote_hip_dequantize_q4_k_f32(const void* weights, void* output, uint64_t rows,
                                 uint64_t input_features, void* stream);
int mote_hip_dequantize_q6_k_f32(const void* weights, void* output, uint64_t rows,
                                 uint64_t input_features, void* stream);

/* ---- Q4_0 dispatch context (per-(M, N, K) plan cache) -------------------- */
/* [new] Handle pattern of the reference's hipBLASLt plan cache
 * (crates/mote-backend-hip/src/hipblaslt_shim.cpp:326-408): create / destroy
 * / last_error, a mutex-guarded map from (M, N, K, op, output type) to the
 * kernel variant, chosen on first use by a shape heuristic or, with autotune
 * on, by timing every eligible variant and the heuristic's own pick on the
 * caller's stream.  Statuses are
 * hipError_t values; on failure last_error describes the cause. */
int mote_q4_0_dispatch_create(void** handle);
void mote_q4_0_dispatch_destroy(void* handle);
const char* mote_q4_0_dispatch_last_error(void* handle);
int mote_q4_0_dispatch_set_autotune(void* handle, int enabled);
/* Split K (K parts of one tile computed by different workgroups): enabled,
 * the tiles kernel adds the parts itself, the last workgroup of a tile to
 * finish summing them in part order (write-through partial stores and a
 * per-tile arrival counter); disabled (the default, faster on MI355X), a
 * second kernel adds them in the same order.  Results are bit-identical. */
int mote_q4_0_dispatch_set_splitk_fold(void* handle, int enabled);
/* Forces one variant by name (NULL or "" clears); tests use it to run every
 * kernel on the same problem. */
int mote_q4_0_dispatch_force_variant(void* handle, const char* name);
int mote_q4_0_dispatch_linear(void* handle, const void* input, const void* weights,
                              void* output, uint64_t rows, uint64_t output_features,
                              uint64_t input_features, int output_f16, void* stream);
int mote_q4_0_dispatch_gate_up_silu(void* handle, const void* input, const void* gate_weights,
                                    const void* up_weights, void* output, uint64_t rows,
                                    uint64_t output_features, uint64_t input_features,
                                    int output_f16, void* stream);
/* The Q8_0 linear through the same context (its own plans and variants). */
int mote_q4_0_dispatch_linear_q8_0(void* handle, const void* input, const void* weights,
                                   void* output, uint64_t rows, uint64_t output_features,
                                   uint64_t input_features, int output_f16, void* stream);
/* Name of the cached variant for a problem (gate_up_op: 0 linear, 1 gate/up,
 * 2 Q8_0 linear); hipErrorNotFound (500) when the problem has not run yet. */
int mote_q4_0_dispatch_plan(void* handle, uint64_t rows, uint64_t output_features,
                            uint64_t input_features, int gate_up_op, int output_f16,
                            char* name, size_t capacity);
/* The variant the context would plan for a problem with 256-byte aligned
 * operands (op: 0 linear, 1 gate/up, 2 Q8_0 linear): the forced variant, else
 * the shape heuristic's choice ("wide_k" for K above 2^31 - 1, which a forced
 * variant cannot run).  Host only: nothing is launched or cached, and no
 * device is needed.  hipErrorInvalidValue (1) for an empty or unsupported
 * shape, hipErrorNotFound (500) when no variant fits. */
int mote_q4_0_dispatch_select(void* handle, uint64_t rows, uint64_t output_features,
                              uint64_t input_features, int op, char* name, size_t capacity);
/* No counterpart in the reference (for the plan-table benchmark, bench.py
 * --plan-table): the comma-separated names of the variants the autotuner
 * would time for a problem with 256-byte aligned operands, the rule-based
 * heuristic's pick included.  Host only.  hipErrorInvalidValue (1) for an
 * empty or unsupported shape or a buffer too small for the list. */
int mote_q4_0_dispatch_candidates(void* handle, uint64_t rows, uint64_t output_features,
                                  uint64_t input_features, int op, char* names, size_t capacity);
int mote_q4_0_variant_count(void);
const char* mote_q4_0_variant_name(int index);

/* ---- Dense F16 x F16 -> F32 matmul (hipBLASLt) ---------------------------- */
/* [reference] crates/mote-backend-hip/src/hipblaslt_shim.cpp:326-408, bound at
 * crates/mote-backend-hip/src/ffi.rs:329-417 for matmul_f16_f32
 * (crates/mote-backend-hip/src/matmul.rs:10-52).  Row-major C[m, n] (f32) =
 * A[m, k] B[k, n] (f16), f32 accumulation, on `stream`, with a caller-owned
 * workspace (the reference passes 32 MiB).  A context caches one plan per
 * (m, n, k); the first call for a shape times hipBLASLt's heuristic
 * candidates on the stream (synchronising it) and keeps the fastest.
 * Statuses: 0; -1 for a null argument or an internal error; hipBLAS
 * statuses from the library; -1000 - hipError for HIP runtime failures;
 * last_error describes the most recent failure ("" after a success).
 * m == 0 or n == 0 returns 0 without a launch; k == 0 writes zeros. */
int mote_hipblaslt_create(void** handle);
void mote_hipblaslt_destroy(void* handle);
const char* mote_hipblaslt_last_error(void* handle);
int mote_hipblaslt_matmul_f16_f32(void* handle, uint64_t m, uint64_t n, uint64_t k, const void* lhs,
                                  const void* rhs, void* output, void* workspace, size_t workspace_bytes,
                                  void* stream);

/* ---- RMSNorm and fused add + RMSNorm -------------------------------------- */
/* [reference] crates/mote-backend-hip/src/rms_norm.hip:68-98, bound at
 * crates/mote-backend-hip/src/ffi.rs:120-161.  f16 [rows, hidden] in/out,
 * f16 weight [hidden], f32 arithmetic.  -1 for null pointers or rows >
 * UINT32_MAX; rows == 0 or hidden == 0 -> 0 without a launch. */
int mote_hip_rms_norm_f16(const void* input, const void* weight, void* output, uint64_t rows,
                          uint64_t hidden_size, float epsilon, void* stream);

/* [reference] crates/mote-backend-hip/src/fused_add_rms_norm.hip:99-138,
 * bound at crates/mote-backend-hip/src/ffi.rs:163-219.  s = input + residual
 * in f32; output = f16(s * rsqrt(mean(s^2) + eps) * weight); residual <-
 * f16(s).  input may alias output; output == residual, a non-finite or
 * negative epsilon, null pointers or rows > UINT32_MAX -> -1. */
int mote_hip_fused_add_rms_norm_f16(const void* input, void* residual, const void* weight,
                                    void* output, uint64_t rows, uint64_t hidden_size,
                                    float epsilon, void* stream);

/* ---- RoPE ------------------------------------------------------------------ */
/* [reference] crates/mote-backend-hip/src/rope.hip:99-150, bound at
 * crates/mote-backend-hip/src/ffi.rs:221-285.  f16 [tokens, heads, head_dim]
 * in/out (may alias), f32 cos/sin [tokens, rotary_dim / 2]; layout 0 =
 * half-split (pairs j, j + R/2), 1 = interleaved (2j, 2j + 1); the tail past
 * rotary_dim is copied.  -1 for null input/output/stream, null cos/sin with
 * rotary_dim > 0, an unknown layout, an odd or oversized rotary_dim, or
 * tokens * heads > UINT32_MAX; any zero dimension -> 0 without a launch. */
int mote_hip_rope_f16(const void* input, const void* cos, const void* sin, void* output,
                      uint64_t tokens, uint64_t heads, uint64_t head_dim, uint64_t rotary_dim,
                      uint32_t layout, void* stream);

/* [new] q and k rotated in one launch with the shared cos/sin rows; same
 * semantics and status codes as mote_hip_rope_f16 applied to each tensor. */
int mote_hip_rope_qk_f16(const void* q_input, const void* k_input, const void* cos,
                         const void* sin, void* q_output, void* k_output, uint64_t tokens,
                         uint64_t q_heads, uint64_t k_heads, uint64_t head_dim,
                         uint64_t rotary_dim, uint32_t layout, void* stream);

/* [new] cos/sin tables [tokens, rotary_dim / 2] from int64 positions:
 * inv_j = theta^(-2j / rotary_dim), angle = position * inv_j, computed in
 * binary64 and rounded to binary32.  -1 for null pointers, an odd rotary_dim
 * or theta <= 0. */
int mote_hip_rope_tables_f32(const void* positions, void* cos_out, void* sin_out,
                             uint64_t tokens, uint64_t rotary_dim, double theta, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOTE_HIP_H */

/*
 * CPU oracle for the Q4_0 quantized-linear path, RMSNorm, fused add + RMSNorm
 * and RoPE.  TEST INFRASTRUCTURE ONLY: the tests, the smoke check and the
 * bench's CPU-baseline leg use it as the checker; nothing in the product
 * (mote_amd/) links, imports or calls it.
 *
 * Each function restates the pure-Rust reference oracle (`mote-reference`)
 * and cites the file:line it follows.  The f32 functions perform the same
 * IEEE-754 operations in the same order as the Rust code (the library is
 * compiled with -ffp-contract=off and without fast-math, and Rust never
 * contracts a*b+c into an FMA), so they are bit-identical restatements.  The
 * f64 functions are the parity judge for the linear: every product of an f16
 * activation and a decoded Q4_0 weight is exact in binary64, so only the
 * summation rounds.
 *
 * Error codes mirror the Rust error enums variant by variant; `detail`
 * receives the variant's fields (expected/actual, rows/..., etc.).
 */
#ifndef MOTE_ORACLE_H
#define MOTE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* mote_types::QuantFormat, in declaration order (TYP/src/lib.rs:41-46). */
enum {
    MOTE_ORACLE_Q8_0 = 0,
    MOTE_ORACLE_Q4_0 = 1,
    MOTE_ORACLE_Q4_K = 2,
    MOTE_ORACLE_Q6_K = 3,
};

/* mote_reference::QuantizedLinearError (REF/src/quantized.rs:6-44). */
enum {
    MOTE_ORACLE_OK = 0,
    MOTE_ORACLE_UNSUPPORTED_FORMAT = 1,      /* detail[0]=format */
    MOTE_ORACLE_ROW_MISALIGNED = 2,          /* format, row_elements, block_elements */
    MOTE_ORACLE_DIMENSIONS_OVERFLOW = 3,     /* rows, output_features, input_features */
    MOTE_ORACLE_INPUT_LENGTH_MISMATCH = 4,   /* expected, actual */
    MOTE_ORACLE_WEIGHT_LENGTH_MISMATCH = 5,  /* expected, actual */
    MOTE_ORACLE_ROW_BYTE_LENGTH_MISMATCH = 6 /* expected, actual */
};

/* mote_reference::ReferenceError (REF/src/lib.rs:19-58) and RopeError (:76-103). */
enum {
    MOTE_ORACLE_ZERO_HIDDEN_SIZE = 20,
    MOTE_ORACLE_NORM_WEIGHT_LENGTH_MISMATCH = 21, /* weight_len, hidden_size */
    MOTE_ORACLE_INPUT_NOT_MULTIPLE = 22,          /* input_len, hidden_size */
    MOTE_ORACLE_RESIDUAL_LENGTH_MISMATCH = 23,    /* residual_len, input_len */
    MOTE_ORACLE_INVALID_EPSILON = 24,
    MOTE_ORACLE_ODD_ROTARY_DIMENSION = 30,        /* rotary_dim */
    MOTE_ORACLE_ROTARY_DIMENSION_TOO_LARGE = 31,  /* rotary_dim, head_dim */
    MOTE_ORACLE_ROPE_DIMENSIONS_OVERFLOW = 32,
    MOTE_ORACLE_ROPE_INPUT_LENGTH_MISMATCH = 33,  /* expected, actual */
    MOTE_ORACLE_COS_LENGTH_MISMATCH = 34,
    MOTE_ORACLE_SIN_LENGTH_MISMATCH = 35,
    MOTE_ORACLE_MATMUL_DIMENSIONS_OVERFLOW = 40,
    MOTE_ORACLE_LHS_LENGTH_MISMATCH = 41,
    MOTE_ORACLE_RHS_LENGTH_MISMATCH = 42
};

/* mote_types::RopeLayout (TYP/src/lib.rs:82-89). */
enum { MOTE_ORACLE_ROPE_HALF_SPLIT = 0, MOTE_ORACLE_ROPE_INTERLEAVED = 1 };

/* --- IEEE-754 binary16 <-> binary32, from the format definition --------- */
float mote_oracle_f16_to_f32(uint16_t bits);
uint16_t mote_oracle_f32_to_f16(float value); /* round to nearest, ties to even */
void mote_oracle_f16_to_f32_array(const uint16_t* in, float* out, size_t n);
void mote_oracle_f32_to_f16_array(const float* in, uint16_t* out, size_t n);

/* --- block geometry (TYP/src/lib.rs:48-73) ------------------------------- */
size_t mote_oracle_block_elements(int format);
size_t mote_oracle_block_bytes(int format);
size_t mote_oracle_alignment_bytes(int format);

/* --- quantized rows and linear (REF/src/quantized.rs) -------------------- */
int mote_oracle_dequantize_row(const uint8_t* bytes, size_t bytes_len, int format,
                               size_t row_elements, float* out, uint64_t detail[3]);

int mote_oracle_quantized_linear_f32(const float* input, size_t input_len,
                                     const uint8_t* weights, size_t weights_len,
                                     int format, size_t rows, size_t output_features,
                                     size_t input_features, float* out,
                                     uint64_t detail[3]);

/* f64-accumulated judge.  Computes out[r * n_cols + c] for every row r and
 * each listed output feature columns[c] (pass columns=NULL for all N). */
int mote_oracle_quantized_linear_f64(const float* input, const uint8_t* weights,
                                     int format, size_t rows, size_t output_features,
                                     size_t input_features, const uint64_t* columns,
                                     size_t n_cols, double* out);

/* Fused gate/up: out = silu(x.Wg^T) * (x.Wu^T), accumulated in f64. */
int mote_oracle_gate_up_silu_f64(const float* input, const uint8_t* gate,
                                 const uint8_t* up, size_t rows, size_t output_features,
                                 size_t input_features, const uint64_t* columns,
                                 size_t n_cols, double* out);

/* --- K-quant super-blocks (Q4_K, Q6_K) ------------------------------------
 * The reference defines only their geometry (TYP/src/lib.rs:39-74: 256
 * elements in 144 / 210 bytes, "ggml-common.h ABI") and its oracle rejects
 * them (REF/src/quantized.rs:154-156, mirrored by the functions above), so
 * these follow the GGML definition the reference names: ggml-common.h
 * block_q4_K / block_q6_K, decoded as ggml-quants.c dequantize_row_q4_K /
 * dequantize_row_q6_K (ggml is not vendored in the reference and no version
 * is pinned there; the layout below is the QK_K = 256 one).  Parity against
 * the reference is therefore unpinned; the tests pin these functions with
 * hand-derived known-answer blocks, the exact-rational closed form of every
 * element, and a packer that writes blocks from the encoder's side.
 *
 * Q4_K (144 bytes): f16 d, f16 dmin, 12 bytes of 6-bit sub-block scales and
 * mins, 128 bytes of nibbles.  Element 64p + 32h + l (p = 0..3, h = 0..1,
 * l = 0..31) is nibble h of byte qs[32p + l] (h = 0 the low nibble), in
 * sub-block j = 2p + h, value f32(d * sc_j) * q - f32(dmin * m_j), where
 * for j < 4 sc_j = s[j] & 63, m_j = s[j + 4] & 63, and for j >= 4
 * sc_j = (s[j + 4] & 15) | (s[j - 4] >> 6) << 4,
 * m_j = (s[j + 4] >> 4) | (s[j] >> 6) << 4.
 * Q6_K (210 bytes): ql[128] low nibbles, qh[64] high bit pairs, int8
 * scales[16], f16 d.  Element 128g + 32c + l (g = 0..1, c = 0..3,
 * l = 0..31) has q = nibble (c >> 1) of ql[64g + 32(c & 1) + l] plus
 * bits 2c..2c+1 of qh[32g + l] shifted to bits 4..5, value
 * f32(d * scales[e / 16]) * (q - 32). */
int mote_oracle_dequantize_kquant_row(const uint8_t* bytes, size_t bytes_len, int format,
                                      size_t row_elements, float* out);

/* f64 judge of a K-quant linear: out[r * N + n] = sum_k x[r, k] w[n, k] in
 * binary64 over the decoded weights (products exact in binary64). */
int mote_oracle_kquant_linear_f64(const float* input, const uint8_t* weights, int format,
                                  size_t rows, size_t output_features, size_t input_features,
                                  double* out);

/* --- dense matmul (REF/src/lib.rs:116-156) -------------------------------- */
int mote_oracle_matmul_f32(const float* lhs, size_t lhs_len, const float* rhs,
                           size_t rhs_len, size_t m, size_t n, size_t k, float* out,
                           uint64_t detail[3]);

/* --- RoPE (REF/src/lib.rs:170-244) ---------------------------------------- */
int mote_oracle_rope_f32(const float* input, size_t input_len, const float* cos_table,
                         size_t cos_len, const float* sin_table, size_t sin_len,
                         size_t tokens, size_t heads, size_t head_dim, size_t rotary_dim,
                         int layout, float* out, uint64_t detail[3]);

/* cos/sin tables for theta-based RoPE: inv_i = theta^(-2i/rotary_dim),
 * c = f32(cos(pos * inv_i)), s = f32(sin(pos * inv_i)), all in f64.  This
 * table builder has no counterpart in the reference (the reference takes
 * caller-built tables, REF/src/lib.rs:158-163). */
void mote_oracle_rope_tables(const int64_t* positions, size_t tokens, size_t rotary_dim,
                             double theta, float* cos_out, float* sin_out);

/* --- RMSNorm and fused add + RMSNorm (REF/src/lib.rs:262-384) -------------- */
int mote_oracle_rms_norm_f32(const float* input, size_t input_len, const float* weight,
                             size_t weight_len, size_t hidden_size, float epsilon,
                             float* out, uint64_t detail[3]);

int mote_oracle_fused_add_rms_norm_f32(const float* input, size_t input_len,
                                       const float* residual, size_t residual_len,
                                       const float* weight, size_t weight_len,
                                       size_t hidden_size, float epsilon,
                                       float* normalized, float* residual_out,
                                       uint64_t detail[3]);

/* --- CPU baseline timing ------------------------------------------------- */
/* Runs mote_oracle_quantized_linear_f32 `iterations` times and returns the
 * elapsed monotonic seconds. */
double mote_oracle_time_quantized_linear_f32(const float* input, const uint8_t* weights,
                                             size_t rows, size_t output_features,
                                             size_t input_features, float* out,
                                             int iterations);

#ifdef __cplusplus
}
#endif

#endif /* MOTE_ORACLE_H */

/*
 * CPU oracle: a plain-C restatement of `mote-reference` for the Q4_0
 * quantized-linear path and the norms / RoPE beside it.  TEST
 * INFRASTRUCTURE ONLY (see mote_oracle.h); never linked into the product.
 *
 * Build: oracle/Makefile, gcc -O2 -ffp-contract=off (no fast-math), so every
 * f32 expression below rounds exactly where the Rust source rounds.
 */
#define _POSIX_C_SOURCE 199309L
#include "mote_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ------------------------------------------------------------------------ */
/* binary16 <-> binary32 from the IEEE-754 definition.                        */
/* The reference converts scales with half 2.7.1 `f16::from_bits(..).to_f32()` */
/* (REF/src/quantized.rs:181) and rounds test data with `f16::from_f32`.      */
/* ------------------------------------------------------------------------ */

float mote_oracle_f16_to_f32(uint16_t bits) {
    const uint32_t sign = (uint32_t)(bits >> 15);
    const uint32_t exponent = (uint32_t)(bits >> 10) & 0x1fu;
    const uint32_t mantissa = (uint32_t)bits & 0x3ffu;
    float magnitude;
    if (exponent == 0) {
        /* zero or subnormal: mantissa * 2^-24, exact in binary32 */
        magnitude = ldexpf((float)mantissa, -24);
    } else if (exponent == 31) {
        if (mantissa == 0) {
            magnitude = INFINITY;
        } else {
            /* NaN: quiet bit set, payload kept in the top mantissa bits */
            uint32_t out = (sign << 31) | 0x7fc00000u | (mantissa << 13);
            float f;
            memcpy(&f, &out, sizeof f);
            return f;
        }
    } else {
        /* normal: (1024 + mantissa) * 2^(exponent - 25), exact */
        magnitude = ldexpf((float)(1024u + mantissa), (int)exponent - 25);
    }
    return sign ? -magnitude : magnitude;
}

uint16_t mote_oracle_f32_to_f16(float value) {
    uint32_t x;
    memcpy(&x, &value, sizeof x);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) {
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) { /* >= 65520 rounds to infinity */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax >= 0x38800000u) { /* >= 2^-14: normal binary16 */
        const uint32_t exponent = (ax >> 23) - 127u + 15u;
        const uint32_t mantissa = ax & 0x7fffffu;
        uint32_t h = (exponent << 10) | (mantissa >> 13);
        const uint32_t rem = mantissa & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) {
            h += 1u; /* a carry into the exponent is the correct result */
        }
        return (uint16_t)(sign | h);
    }
    /* subnormal binary16 (units of 2^-24) or zero */
    const uint32_t exponent_field = ax >> 23;
    if (exponent_field == 0) {
        return sign; /* binary32 subnormals are far below 2^-25 */
    }
    const uint32_t significand = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - exponent_field; /* >= 14 here */
    if (shift >= 25u) {
        return sign; /* below half of the smallest subnormal */
    }
    uint32_t m = significand >> shift;
    const uint32_t rem = significand & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (m & 1u))) {
        m += 1u;
    }
    return (uint16_t)(sign | m);
}

void mote_oracle_f16_to_f32_array(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = mote_oracle_f16_to_f32(in[i]);
}

void mote_oracle_f32_to_f16_array(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = mote_oracle_f32_to_f16(in[i]);
}

/* ------------------------------------------------------------------------ */
/* Geometry: TYP/src/lib.rs:48-73                                             */
/* ------------------------------------------------------------------------ */

size_t mote_oracle_block_elements(int format) {
    switch (format) {
        case MOTE_ORACLE_Q4_0:
        case MOTE_ORACLE_Q8_0: return 32;
        case MOTE_ORACLE_Q4_K:
        case MOTE_ORACLE_Q6_K: return 256;
        default: return 0;
    }
}

size_t mote_oracle_block_bytes(int format) {
    switch (format) {
        case MOTE_ORACLE_Q4_0: return 18;
        case MOTE_ORACLE_Q8_0: return 34;
        case MOTE_ORACLE_Q4_K: return 144;
        case MOTE_ORACLE_Q6_K: return 210;
        default: return 0;
    }
}

size_t mote_oracle_alignment_bytes(int format) {
    switch (format) {
        case MOTE_ORACLE_Q4_0:
        case MOTE_ORACLE_Q8_0:
        case MOTE_ORACLE_Q6_K: return 2;
        case MOTE_ORACLE_Q4_K: return 4;
        default: return 0;
    }
}

static void set_detail(uint64_t detail[3], uint64_t a, uint64_t b, uint64_t c) {
    if (detail) {
        detail[0] = a;
        detail[1] = b;
        detail[2] = c;
    }
}

/* checked_row_bytes: REF/src/quantized.rs:146-175 */
static int checked_row_bytes(int format, size_t row_elements, size_t rows,
                             size_t output_features, size_t* row_bytes,
                             uint64_t detail[3]) {
    if (format != MOTE_ORACLE_Q4_0 && format != MOTE_ORACLE_Q8_0) {
        set_detail(detail, (uint64_t)format, 0, 0);
        return MOTE_ORACLE_UNSUPPORTED_FORMAT;
    }
    const size_t block_elements = mote_oracle_block_elements(format);
    if (row_elements % block_elements != 0) {
        set_detail(detail, (uint64_t)format, row_elements, block_elements);
        return MOTE_ORACLE_ROW_MISALIGNED;
    }
    if (__builtin_mul_overflow(row_elements / block_elements,
                               mote_oracle_block_bytes(format), row_bytes)) {
        set_detail(detail, rows, output_features, row_elements);
        return MOTE_ORACLE_DIMENSIONS_OVERFLOW;
    }
    return MOTE_ORACLE_OK;
}

/* decode_row_into: REF/src/quantized.rs:177-201 */
static void decode_row_into(const uint8_t* bytes, size_t row_bytes, int format, float* out) {
    const size_t block_bytes = mote_oracle_block_bytes(format);
    const size_t block_elements = mote_oracle_block_elements(format);
    for (size_t b = 0; b * block_bytes < row_bytes; ++b) {
        const uint8_t* block = bytes + b * block_bytes;
        const float scale = mote_oracle_f16_to_f32((uint16_t)(block[0] | (block[1] << 8)));
        float* o = out + b * block_elements;
        if (format == MOTE_ORACLE_Q4_0) {
            for (int j = 0; j < 16; ++j) {
                const uint8_t quants = block[2 + j];
                o[j] = (float)((int8_t)(quants & 0x0f) - 8) * scale;
                o[j + 16] = (float)((int8_t)(quants >> 4) - 8) * scale;
            }
        } else {
            for (int j = 0; j < 32; ++j) {
                o[j] = (float)(int8_t)block[2 + j] * scale;
            }
        }
    }
}

/* dequantize_quantized_row: REF/src/quantized.rs:58-74 */
int mote_oracle_dequantize_row(const uint8_t* bytes, size_t bytes_len, int format,
                               size_t row_elements, float* out, uint64_t detail[3]) {
    size_t row_bytes = 0;
    int status = checked_row_bytes(format, row_elements, 1, 1, &row_bytes, detail);
    if (status != MOTE_ORACLE_OK) return status;
    if (bytes_len != row_bytes) {
        set_detail(detail, row_bytes, bytes_len, 0);
        return MOTE_ORACLE_ROW_BYTE_LENGTH_MISMATCH;
    }
    if (row_elements) decode_row_into(bytes, row_bytes, format, out);
    return MOTE_ORACLE_OK;
}

/* ------------------------------------------------------------------------ */
/* K-quant super-blocks: GGML's block_q4_K / block_q6_K (ggml-common.h) and  */
/* dequantize_row_q4_K / dequantize_row_q6_K (ggml-quants.c); the reference  */
/* has their geometry only (TYP/src/lib.rs:39-74).  Element order and f32   */
/* rounding points as GGML's C: d1 = d * sc and m1 = dmin * m rounded to f32, */
/* then d1 * q - m1 (Q4_K); d * sc then times (q - 32) (Q6_K).              */
/* ------------------------------------------------------------------------ */

/* get_scale_min_k4 of ggml-quants.c: 6-bit scale and min of sub-block j. */
static void q4k_scale_min(const uint8_t* s, int j, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

static void decode_q4_k_block(const uint8_t* b, float* y) {
    const float d = mote_oracle_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
    const float dmin = mote_oracle_f16_to_f32((uint16_t)(b[2] | (b[3] << 8)));
    const uint8_t* s = b + 4;
    const uint8_t* q = b + 16;
    for (int p = 0; p < 4; ++p) {
        for (int h = 0; h < 2; ++h) {
            uint8_t sc, m;
            q4k_scale_min(s, 2 * p + h, &sc, &m);
            const float d1 = d * (float)sc;
            const float m1 = dmin * (float)m;
            for (int l = 0; l < 32; ++l) {
                const int nib = h ? (q[32 * p + l] >> 4) : (q[32 * p + l] & 0x0f);
                const float prod = d1 * (float)nib;
                y[64 * p + 32 * h + l] = prod - m1;
            }
        }
    }
}

static void decode_q6_k_block(const uint8_t* b, float* y) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    const float d = mote_oracle_f16_to_f32((uint16_t)(b[208] | (b[209] << 8)));
    for (int g = 0; g < 2; ++g) {
        for (int c = 0; c < 4; ++c) {
            for (int l = 0; l < 32; ++l) {
                const int e = 128 * g + 32 * c + l;
                const uint8_t lowbyte = ql[64 * g + 32 * (c & 1) + l];
                const int low = (c >> 1) ? (lowbyte >> 4) : (lowbyte & 0x0f);
                const int high = (qh[32 * g + l] >> (2 * c)) & 3;
                const int q = (low | (high << 4)) - 32;
                const float ds = d * (float)sc[e / 16];
                y[e] = ds * (float)q;
            }
        }
    }
}

int mote_oracle_dequantize_kquant_row(const uint8_t* bytes, size_t bytes_len, int format,
                                      size_t row_elements, float* out) {
    if (format != MOTE_ORACLE_Q4_K && format != MOTE_ORACLE_Q6_K) return MOTE_ORACLE_UNSUPPORTED_FORMAT;
    if (row_elements % 256 != 0) return MOTE_ORACLE_ROW_MISALIGNED;
    const size_t block_bytes = mote_oracle_block_bytes(format);
    if (bytes_len != row_elements / 256 * block_bytes) return MOTE_ORACLE_ROW_BYTE_LENGTH_MISMATCH;
    for (size_t b = 0; b < row_elements / 256; ++b) {
        if (format == MOTE_ORACLE_Q4_K)
            decode_q4_k_block(bytes + b * block_bytes, out + 256 * b);
        else
            decode_q6_k_block(bytes + b * block_bytes, out + 256 * b);
    }
    return MOTE_ORACLE_OK;
}

int mote_oracle_kquant_linear_f64(const float* input, const uint8_t* weights, int format,
                                  size_t rows, size_t output_features, size_t input_features,
                                  double* out) {
    if (format != MOTE_ORACLE_Q4_K && format != MOTE_ORACLE_Q6_K) return MOTE_ORACLE_UNSUPPORTED_FORMAT;
    if (input_features % 256 != 0) return MOTE_ORACLE_ROW_MISALIGNED;
    const size_t row_bytes = input_features / 256 * mote_oracle_block_bytes(format);
    float* w = (float*)malloc((input_features ? input_features : 1) * sizeof(float));
    if (!w) return -1;
    for (size_t n = 0; n < output_features; ++n) {
        mote_oracle_dequantize_kquant_row(weights + n * row_bytes, row_bytes, format, input_features, w);
        for (size_t r = 0; r < rows; ++r) {
            const float* x = input + r * input_features;
            double acc = 0.0;
            for (size_t k = 0; k < input_features; ++k) acc += (double)x[k] * (double)w[k];
            out[r * output_features + n] = acc;
        }
    }
    free(w);
    return MOTE_ORACLE_OK;
}

/* quantized_linear_f32: REF/src/quantized.rs:89-144.  Same loop order: decode
 * one weight row, then a sequential f32 multiply-then-add over K per row. */
int mote_oracle_quantized_linear_f32(const float* input, size_t input_len,
                                     const uint8_t* weights, size_t weights_len,
                                     int format, size_t rows, size_t output_features,
                                     size_t input_features, float* out,
                                     uint64_t detail[3]) {
    size_t row_bytes = 0, in_len = 0, w_len = 0, out_len = 0;
    int status = checked_row_bytes(format, input_features, rows, output_features,
                                   &row_bytes, detail);
    if (status != MOTE_ORACLE_OK) return status;
    if (__builtin_mul_overflow(rows, input_features, &in_len) ||
        __builtin_mul_overflow(output_features, row_bytes, &w_len) ||
        __builtin_mul_overflow(rows, output_features, &out_len)) {
        set_detail(detail, rows, output_features, input_features);
        return MOTE_ORACLE_DIMENSIONS_OVERFLOW;
    }
    if (input_len != in_len) {
        set_detail(detail, in_len, input_len, 0);
        return MOTE_ORACLE_INPUT_LENGTH_MISMATCH;
    }
    if (weights_len != w_len) {
        set_detail(detail, w_len, weights_len, 0);
        return MOTE_ORACLE_WEIGHT_LENGTH_MISMATCH;
    }
    if (out_len == 0) return MOTE_ORACLE_OK;

    float* decoded = (float*)malloc((input_features ? input_features : 1) * sizeof(float));
    if (!decoded) return -1;
    for (size_t n = 0; n < output_features; ++n) {
        decode_row_into(weights + n * row_bytes, row_bytes, format, decoded);
        for (size_t r = 0; r < rows; ++r) {
            const float* x = input + r * input_features;
            float sum = 0.0f;
            for (size_t k = 0; k < input_features; ++k) {
                sum += x[k] * decoded[k];
            }
            out[r * output_features + n] = sum;
        }
    }
    free(decoded);
    return MOTE_ORACLE_OK;
}

static int linear_f64_columns(const float* input, const uint8_t* weights, int format,
                              size_t rows, size_t output_features, size_t input_features,
                              const uint64_t* columns, size_t n_cols, double* out,
                              const uint8_t* second, int gate_up) {
    size_t row_bytes = 0;
    int status = checked_row_bytes(format, input_features, rows, output_features,
                                   &row_bytes, NULL);
    if (status != MOTE_ORACLE_OK) return status;
    const size_t count = columns ? n_cols : output_features;
    float* a = (float*)malloc((input_features ? input_features : 1) * sizeof(float));
    float* b = (float*)malloc((input_features ? input_features : 1) * sizeof(float));
    if (!a || !b) {
        free(a);
        free(b);
        return -1;
    }
    for (size_t c = 0; c < count; ++c) {
        const size_t n = columns ? (size_t)columns[c] : c;
        if (n >= output_features) {
            free(a);
            free(b);
            return -2;
        }
        decode_row_into(weights + n * row_bytes, row_bytes, format, a);
        if (gate_up) decode_row_into(second + n * row_bytes, row_bytes, format, b);
        for (size_t r = 0; r < rows; ++r) {
            const float* x = input + r * input_features;
            double g = 0.0, u = 0.0;
            for (size_t k = 0; k < input_features; ++k) {
                g += (double)x[k] * (double)a[k];
                if (gate_up) u += (double)x[k] * (double)b[k];
            }
            out[r * count + c] = gate_up ? (g / (1.0 + exp(-g))) * u : g;
        }
    }
    free(a);
    free(b);
    return MOTE_ORACLE_OK;
}

int mote_oracle_quantized_linear_f64(const float* input, const uint8_t* weights,
                                     int format, size_t rows, size_t output_features,
                                     size_t input_features, const uint64_t* columns,
                                     size_t n_cols, double* out) {
    return linear_f64_columns(input, weights, format, rows, output_features,
                              input_features, columns, n_cols, out, NULL, 0);
}

int mote_oracle_gate_up_silu_f64(const float* input, const uint8_t* gate,
                                 const uint8_t* up, size_t rows, size_t output_features,
                                 size_t input_features, const uint64_t* columns,
                                 size_t n_cols, double* out) {
    return linear_f64_columns(input, gate, MOTE_ORACLE_Q4_0, rows, output_features,
                              input_features, columns, n_cols, out, up, 1);
}

/* matmul_f32: REF/src/lib.rs:116-156 */
int mote_oracle_matmul_f32(const float* lhs, size_t lhs_len, const float* rhs,
                           size_t rhs_len, size_t m, size_t n, size_t k, float* out,
                           uint64_t detail[3]) {
    size_t l = 0, r = 0, o = 0;
    if (__builtin_mul_overflow(m, k, &l) || __builtin_mul_overflow(k, n, &r) ||
        __builtin_mul_overflow(m, n, &o)) {
        set_detail(detail, m, n, k);
        return MOTE_ORACLE_MATMUL_DIMENSIONS_OVERFLOW;
    }
    if (lhs_len != l) {
        set_detail(detail, l, lhs_len, 0);
        return MOTE_ORACLE_LHS_LENGTH_MISMATCH;
    }
    if (rhs_len != r) {
        set_detail(detail, r, rhs_len, 0);
        return MOTE_ORACLE_RHS_LENGTH_MISMATCH;
    }
    for (size_t i = 0; i < o; ++i) out[i] = 0.0f;
    for (size_t row = 0; row < m; ++row) {
        for (size_t inner = 0; inner < k; ++inner) {
            const float lv = lhs[row * k + inner];
            for (size_t col = 0; col < n; ++col) {
                out[row * n + col] += lv * rhs[inner * n + col];
            }
        }
    }
    return MOTE_ORACLE_OK;
}

/* rope_f32: REF/src/lib.rs:170-244 */
int mote_oracle_rope_f32(const float* input, size_t input_len, const float* cos_table,
                         size_t cos_len, const float* sin_table, size_t sin_len,
                         size_t tokens, size_t heads, size_t head_dim, size_t rotary_dim,
                         int layout, float* out, uint64_t detail[3]) {
    if (rotary_dim % 2 != 0) {
        set_detail(detail, rotary_dim, 0, 0);
        return MOTE_ORACLE_ODD_ROTARY_DIMENSION;
    }
    if (rotary_dim > head_dim) {
        set_detail(detail, rotary_dim, head_dim, 0);
        return MOTE_ORACLE_ROTARY_DIMENSION_TOO_LARGE;
    }
    size_t rows = 0, in_len = 0, cache_len = 0;
    const size_t frequency_count = rotary_dim / 2;
    if (__builtin_mul_overflow(tokens, heads, &rows) ||
        __builtin_mul_overflow(rows, head_dim, &in_len) ||
        __builtin_mul_overflow(tokens, frequency_count, &cache_len)) {
        set_detail(detail, tokens, heads, head_dim);
        return MOTE_ORACLE_ROPE_DIMENSIONS_OVERFLOW;
    }
    if (input_len != in_len) {
        set_detail(detail, in_len, input_len, 0);
        return MOTE_ORACLE_ROPE_INPUT_LENGTH_MISMATCH;
    }
    if (cos_len != cache_len) {
        set_detail(detail, cache_len, cos_len, 0);
        return MOTE_ORACLE_COS_LENGTH_MISMATCH;
    }
    if (sin_len != cache_len) {
        set_detail(detail, cache_len, sin_len, 0);
        return MOTE_ORACLE_SIN_LENGTH_MISMATCH;
    }
    if (in_len) memcpy(out, input, in_len * sizeof(float));
    for (size_t t = 0; t < tokens; ++t) {
        const size_t cache_offset = t * frequency_count;
        for (size_t h = 0; h < heads; ++h) {
            const size_t row_offset = (t * heads + h) * head_dim;
            for (size_t p = 0; p < frequency_count; ++p) {
                size_t first, second;
                if (layout == MOTE_ORACLE_ROPE_HALF_SPLIT) {
                    first = p;
                    second = p + frequency_count;
                } else {
                    first = 2 * p;
                    second = 2 * p + 1;
                }
                const float a = input[row_offset + first];
                const float b = input[row_offset + second];
                const float c = cos_table[cache_offset + p];
                const float s = sin_table[cache_offset + p];
                out[row_offset + first] = a * c - b * s;
                out[row_offset + second] = b * c + a * s;
            }
        }
    }
    return MOTE_ORACLE_OK;
}

void mote_oracle_rope_tables(const int64_t* positions, size_t tokens, size_t rotary_dim,
                             double theta, float* cos_out, float* sin_out) {
    const size_t half = rotary_dim / 2;
    for (size_t t = 0; t < tokens; ++t) {
        for (size_t i = 0; i < half; ++i) {
            const double inv = pow(theta, -(2.0 * (double)i) / (double)rotary_dim);
            const double angle = (double)positions[t] * inv;
            cos_out[t * half + i] = (float)cos(angle);
            sin_out[t * half + i] = (float)sin(angle);
        }
    }
}

static int norm_checks(size_t input_len, size_t weight_len, size_t hidden_size,
                       float epsilon, uint64_t detail[3]) {
    if (hidden_size == 0) return MOTE_ORACLE_ZERO_HIDDEN_SIZE;
    if (weight_len != hidden_size) {
        set_detail(detail, weight_len, hidden_size, 0);
        return MOTE_ORACLE_NORM_WEIGHT_LENGTH_MISMATCH;
    }
    (void)input_len;
    (void)epsilon;
    return MOTE_ORACLE_OK;
}

static int epsilon_check(float epsilon) {
    return (!isfinite(epsilon) || epsilon < 0.0f) ? MOTE_ORACLE_INVALID_EPSILON
                                                  : MOTE_ORACLE_OK;
}

static void rms_rows(const float* rows_in, size_t len, const float* weight,
                     size_t hidden_size, float epsilon, float* out) {
    for (size_t start = 0; start < len; start += hidden_size) {
        const float* row = rows_in + start;
        float sum_sq = 0.0f;
        for (size_t i = 0; i < hidden_size; ++i) sum_sq += row[i] * row[i];
        const float mean_square = sum_sq / (float)hidden_size;
        const float inv_rms = 1.0f / sqrtf(mean_square + epsilon);
        for (size_t i = 0; i < hidden_size; ++i) {
            out[start + i] = row[i] * inv_rms * weight[i];
        }
    }
}

/* rms_norm_f32: REF/src/lib.rs:262-301 */
int mote_oracle_rms_norm_f32(const float* input, size_t input_len, const float* weight,
                             size_t weight_len, size_t hidden_size, float epsilon,
                             float* out, uint64_t detail[3]) {
    int status = norm_checks(input_len, weight_len, hidden_size, epsilon, detail);
    if (status != MOTE_ORACLE_OK) return status;
    if (input_len % hidden_size != 0) {
        set_detail(detail, input_len, hidden_size, 0);
        return MOTE_ORACLE_INPUT_NOT_MULTIPLE;
    }
    status = epsilon_check(epsilon);
    if (status != MOTE_ORACLE_OK) return status;
    rms_rows(input, input_len, weight, hidden_size, epsilon, out);
    return MOTE_ORACLE_OK;
}

/* fused_add_rms_norm_f32: REF/src/lib.rs:333-384 */
int mote_oracle_fused_add_rms_norm_f32(const float* input, size_t input_len,
                                       const float* residual, size_t residual_len,
                                       const float* weight, size_t weight_len,
                                       size_t hidden_size, float epsilon,
                                       float* normalized, float* residual_out,
                                       uint64_t detail[3]) {
    int status = norm_checks(input_len, weight_len, hidden_size, epsilon, detail);
    if (status != MOTE_ORACLE_OK) return status;
    if (residual_len != input_len) {
        set_detail(detail, residual_len, input_len, 0);
        return MOTE_ORACLE_RESIDUAL_LENGTH_MISMATCH;
    }
    if (input_len % hidden_size != 0) {
        set_detail(detail, input_len, hidden_size, 0);
        return MOTE_ORACLE_INPUT_NOT_MULTIPLE;
    }
    status = epsilon_check(epsilon);
    if (status != MOTE_ORACLE_OK) return status;
    for (size_t i = 0; i < input_len; ++i) residual_out[i] = input[i] + residual[i];
    rms_rows(residual_out, input_len, weight, hidden_size, epsilon, normalized);
    return MOTE_ORACLE_OK;
}

double mote_oracle_time_quantized_linear_f32(const float* input, const uint8_t* weights,
                                             size_t rows, size_t output_features,
                                             size_t input_features, float* out,
                                             int iterations) {
    const size_t row_bytes = (input_features / 32) * 18;
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (int i = 0; i < iterations; ++i) {
        mote_oracle_quantized_linear_f32(input, rows * input_features, weights,
                                         output_features * row_bytes, MOTE_ORACLE_Q4_0,
                                         rows, output_features, input_features, out, NULL);
    }
    clock_gettime(CLOCK_MONOTONIC, &t1);
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}

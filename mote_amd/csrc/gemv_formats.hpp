// Weight formats of the vector-ALU decode GEMVs (q4_0_gemv_stream.hip,
// q4_0_gemv_lds.hip), shared so that every kernel built on them computes the
// same sums bit for bit: the order x takes in registers, how a block pair's
// quantized values are read as binary16 subnormals, and the order of the dot
// chains.
#pragma once

#include "common.hpp"
#include "q4_0.hpp"

namespace mote::q4_0 {
namespace {

constexpr uint32_t kSubLo = 0x000F000Fu;  // low nibbles of bytes 0 and 2: n * 2^-24
constexpr uint32_t kSubHi = 0x00F000F0u;  // high nibbles of bytes 0 and 2: n * 2^-20

__device__ __forceinline__ uint32_t pick(const uint32_t* x, int a, int b) {
    const uint32_t lo = (a & 1) ? 0x0302u : 0x0100u;
    const uint32_t hi = (b & 1) ? 0x07060000u : 0x05040000u;
    return __builtin_amdgcn_perm(x[b >> 1], x[a >> 1], hi | lo);
}

struct XPair {
    uint32_t xp[32];
    float c0, c1;  // start values of the two blocks' sums (format's kStart times sum of x)
};

// ---------------------------------------------------------------------------
// Rows whose sum is not finite.
//
// The dot chains below multiply a block's scale into the block's sum,
// d * sum x (n - 8); the reference multiplies it into every element first,
// v = (n - 8) d, and then sums x v (crates/mote-reference/src/quantized.rs:
// 181,187-188; Q8_0 v d at :191-195).  For finite scales and activations the
// two agree to rounding: no intermediate of either can overflow (|x v| <=
// 65504 * 128 * 65504 per element).  They part only when a scale is infinite
// or an activation is not finite: with d = inf the reference's v is NaN for
// n = 8 and x v is NaN for x = 0, and products of both signs give
// inf - inf = NaN, where d * sum is +-inf unless the sum is 0.  In every such
// case the factored sum is itself not finite, so a wave whose reduced row (or
// row-slice) sum is not finite -- a test of the wave-uniform value on the
// scalar unit -- recomputes its share of the row element by element with the
// reference's operations (exact_pair below), and the NaN and infinities land
// where the reference puts them.  Ordinary weights never take that branch.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool not_finite(float v) {
    return (__builtin_bit_cast(uint32_t, v) & 0x7F800000u) == 0x7F800000u;
}

__device__ __forceinline__ float f16_bits_to_float(uint16_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

// sum over the 64 elements of the Q4_0 block pair at `pair` (global memory,
// 2-byte aligned) of x * ((n - 8) d), each product and sum in f32: the
// reference's per-element arithmetic.  Rolled loops: the code only runs for
// rows that hold a non-finite scale or activation.
__device__ inline float q4_0_exact_pair(const uint8_t* pair, const uint16_t* x) {
    float acc = 0.0f;
#pragma unroll 1
    for (int b = 0; b < 2; ++b) {
        const uint8_t* blk = pair + 18 * b;
        const float d = f16_bits_to_float(*reinterpret_cast<const uint16_t*>(blk));
#pragma unroll 1
        for (int j = 0; j < 16; ++j) {
            const uint32_t q = blk[2 + j];
            const float lo = static_cast<float>(static_cast<int>(q & 15u) - 8) * d;
            const float hi = static_cast<float>(static_cast<int>(q >> 4) - 8) * d;
            acc += f16_bits_to_float(x[32 * b + j]) * lo;
            acc += f16_bits_to_float(x[32 * b + 16 + j]) * hi;
        }
    }
    return acc;
}

// The same for a Q8_0 block pair (two 34-byte blocks, value v d).
__device__ inline float q8_0_exact_pair(const uint8_t* pair, const uint16_t* x) {
    float acc = 0.0f;
#pragma unroll 1
    for (int b = 0; b < 2; ++b) {
        const uint8_t* blk = pair + 34 * b;
        const float d = f16_bits_to_float(*reinterpret_cast<const uint16_t*>(blk));
#pragma unroll 1
        for (int j = 0; j < 32; ++j)
            acc += f16_bits_to_float(x[32 * b + j]) * (static_cast<float>(static_cast<int8_t>(blk[2 + j])) * d);
    }
    return acc;
}

// Operands of a pair unpacked once and shared by every token of a row.
struct Unpacked {
    uint32_t u[32];
    float d0, d1;
};

// ---------------------------------------------------------------------------
// GGML Q4_0: a pair is two 18-byte blocks (36 bytes, 9 dwords), value
// (n - 8) d.  Nibbles are read as binary16 subnormals, with no carrier term
// and no shift for bytes 0 and 2 of a dword: q & 0x000F000F holds (n_b0,
// n_b2) * 2^-24 and q & 0x00F000F0 holds (n_b0, n_b2) * 2^-20 (the high
// nibbles); bytes 1 and 3 take one shift by 8.  Each such value times an f16
// activation is exact in f32 (v_dot2_f32_f16 honours f16 subnormals: the
// kernels run with f16 denormals enabled), so per block
//   sum x (n - 8) = 2^20 (16 a_lo + a_hi)   with a_hi started at -8 * 2^-20 sum x,
// five VALU operations per nibble dword instead of a mask, shift and OR per
// nibble pair.
// ---------------------------------------------------------------------------
struct FmtQ4 {
    static constexpr uint32_t kPairBytes = 36;
    static constexpr int kDwords = 9;
    static constexpr float kFinal = 1048576.0f;           // 2^20
    static constexpr float kStart = -8.0f / 1048576.0f;   // times the block's sum of x

    __device__ static void load(const uint8_t* p, uint32_t (&d)[kDwords]) { load_pair(p, d); }

    __device__ static float exact(const uint8_t* pair, const uint16_t* x) { return q4_0_exact_pair(pair, x); }

    // x of the pair (64 halves in xr) in the order the nibble operands take it.
    __device__ static void order_x(const uint32_t (&xr)[32], XPair& xv) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int base = (q < 4) ? 0 : 32;
            const int e0 = base + pair_byte_element(q, 0);
            const int e1 = base + pair_byte_element(q, 1);
            const int e2 = base + pair_byte_element(q, 2);
            const int e3 = base + pair_byte_element(q, 3);
            xv.xp[4 * q + 0] = pick(xr, e0 + 16, e2 + 16);  // hi02
            xv.xp[4 * q + 1] = pick(xr, e0, e2);            // lo02
            xv.xp[4 * q + 2] = pick(xr, e1, e3);            // lo13
            xv.xp[4 * q + 3] = pick(xr, e1 + 16, e3 + 16);  // hi13
        }
    }

    // sum_k x_k (n_k - 8) d of the two blocks of a pair, divided by 2^20.
    __device__ static float dot(const uint32_t (&raw)[kDwords], const XPair& x) {
        uint32_t q[8];
        q[0] = pair_q0(raw);
        q[1] = raw[1]; q[2] = raw[2]; q[3] = raw[3];
        q[4] = raw[5]; q[5] = raw[6]; q[6] = raw[7]; q[7] = raw[8];
        const float d0 = half_lo_to_float(raw[0]);
        const float d1 = half_hi_to_float(raw[4]);
        float lo0 = 0.0f, hi0 = x.c0, lo1 = 0.0f, hi1 = x.c1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t a = q[i], b = q[4 + i];
            const uint32_t a8 = a >> 8, b8 = b >> 8;
            hi0 = dot2(a & kSubHi, x.xp[4 * i + 0], hi0);
            lo0 = dot2(a & kSubLo, x.xp[4 * i + 1], lo0);
            lo0 = dot2(a8 & kSubLo, x.xp[4 * i + 2], lo0);
            hi0 = dot2(a8 & kSubHi, x.xp[4 * i + 3], hi0);
            hi1 = dot2(b & kSubHi, x.xp[16 + 4 * i + 0], hi1);
            lo1 = dot2(b & kSubLo, x.xp[16 + 4 * i + 1], lo1);
            lo1 = dot2(b8 & kSubLo, x.xp[16 + 4 * i + 2], lo1);
            hi1 = dot2(b8 & kSubHi, x.xp[16 + 4 * i + 3], hi1);
        }
        const float acc = d0 * __builtin_fmaf(lo0, 16.0f, hi0);
        return __builtin_fmaf(d1, __builtin_fmaf(lo1, 16.0f, hi1), acc);
    }

    // The 32 masked nibble operands in the order of XPair::xp, and the scales.
    __device__ static void unpack(const uint32_t (&raw)[kDwords], Unpacked& o) {
        uint32_t q[8];
        q[0] = pair_q0(raw);
        q[1] = raw[1]; q[2] = raw[2]; q[3] = raw[3];
        q[4] = raw[5]; q[5] = raw[6]; q[6] = raw[7]; q[7] = raw[8];
        o.d0 = half_lo_to_float(raw[0]);
        o.d1 = half_hi_to_float(raw[4]);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t a = q[i], a8 = a >> 8;
            o.u[4 * i + 0] = a & kSubHi;
            o.u[4 * i + 1] = a & kSubLo;
            o.u[4 * i + 2] = a8 & kSubLo;
            o.u[4 * i + 3] = a8 & kSubHi;
        }
    }

    __device__ static float dot(const Unpacked& w, const XPair& x) {
        float lo0 = 0.0f, hi0 = x.c0, lo1 = 0.0f, hi1 = x.c1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            hi0 = dot2(w.u[4 * i + 0], x.xp[4 * i + 0], hi0);
            lo0 = dot2(w.u[4 * i + 1], x.xp[4 * i + 1], lo0);
            lo0 = dot2(w.u[4 * i + 2], x.xp[4 * i + 2], lo0);
            hi0 = dot2(w.u[4 * i + 3], x.xp[4 * i + 3], hi0);
            hi1 = dot2(w.u[16 + 4 * i + 0], x.xp[16 + 4 * i + 0], hi1);
            lo1 = dot2(w.u[16 + 4 * i + 1], x.xp[16 + 4 * i + 1], lo1);
            lo1 = dot2(w.u[16 + 4 * i + 2], x.xp[16 + 4 * i + 2], lo1);
            hi1 = dot2(w.u[16 + 4 * i + 3], x.xp[16 + 4 * i + 3], hi1);
        }
        const float acc = w.d0 * __builtin_fmaf(lo0, 16.0f, hi0);
        return __builtin_fmaf(w.d1, __builtin_fmaf(lo1, 16.0f, hi1), acc);
    }
};

// ---------------------------------------------------------------------------
// GGML Q8_0 (crates/mote-reference/src/quantized.rs:191-195): a block is an
// f16 scale d and 32 two's-complement bytes, value v d; a pair is 68 bytes
// (17 dwords, dword aligned whenever the row is).  Block 0's bytes start at
// pair byte 2, so its dwords are re-aligned with one v_perm each.  XOR 0x80
// turns every byte into u = v + 128; u & 0x00FF00FF read as binary16 is
// (u_b0, u_b2) * 2^-24 exactly (a subnormal), and one shift by 8 gives bytes
// 1 and 3: each product with an f16 activation is exact in f32, so per block
//   sum x v = 2^24 a   with a started at -128 * 2^-24 sum x.
// ---------------------------------------------------------------------------
struct FmtQ8 {
    static constexpr uint32_t kPairBytes = 68;
    static constexpr int kDwords = 17;
    static constexpr float kFinal = 16777216.0f;            // 2^24
    static constexpr float kStart = -128.0f / 16777216.0f;  // times the block's sum of x

    __device__ static void load(const uint8_t* p, uint32_t (&d)[kDwords]) { load_pair_q8(p, d); }

    __device__ static float exact(const uint8_t* pair, const uint16_t* x) { return q8_0_exact_pair(pair, x); }

    // Dword i of the pair's 64 bytes (elements 4i .. 4i + 3) takes x as
    // (x[4i], x[4i + 2]) for bytes 0 and 2 and (x[4i + 1], x[4i + 3]) for 1, 3.
    __device__ static void order_x(const uint32_t (&xr)[32], XPair& xv) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            xv.xp[2 * i + 0] = pick(xr, 4 * i, 4 * i + 2);
            xv.xp[2 * i + 1] = pick(xr, 4 * i + 1, 4 * i + 3);
        }
    }

    __device__ static uint32_t bytes(const uint32_t (&raw)[kDwords], int i) { return q8_bytes(raw, i); }

    __device__ static float dot(const uint32_t (&raw)[kDwords], const XPair& x) {
        float a0 = x.c0, a1 = x.c1;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t u = bytes(raw, i) ^ 0x80808080u;
            const uint32_t w = bytes(raw, 8 + i) ^ 0x80808080u;
            a0 = dot2(u & 0x00FF00FFu, x.xp[2 * i + 0], a0);
            a0 = dot2((u >> 8) & 0x00FF00FFu, x.xp[2 * i + 1], a0);
            a1 = dot2(w & 0x00FF00FFu, x.xp[16 + 2 * i + 0], a1);
            a1 = dot2((w >> 8) & 0x00FF00FFu, x.xp[16 + 2 * i + 1], a1);
        }
        const float d0 = half_lo_to_float(raw[0]);
        const float d1 = half_hi_to_float(raw[8]);
        return __builtin_fmaf(d1, a1, d0 * a0);
    }

    __device__ static void unpack(const uint32_t (&raw)[kDwords], Unpacked& o) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t u = bytes(raw, i) ^ 0x80808080u;
            o.u[2 * i + 0] = u & 0x00FF00FFu;
            o.u[2 * i + 1] = (u >> 8) & 0x00FF00FFu;
        }
        o.d0 = half_lo_to_float(raw[0]);
        o.d1 = half_hi_to_float(raw[8]);
    }

    __device__ static float dot(const Unpacked& w, const XPair& x) {
        float a0 = x.c0, a1 = x.c1;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            a0 = dot2(w.u[i], x.xp[i], a0);
            a1 = dot2(w.u[16 + i], x.xp[16 + i], a1);
        }
        return __builtin_fmaf(w.d1, a1, w.d0 * a0);
    }
};

}  // namespace
}  // namespace mote::q4_0

// Shared device helpers for the gfx950 (CDNA4) kernels of the Q4_0 path.
//
// GGML Q4_0 block (crates/mote-types/src/lib.rs:49-65, decode at
// crates/mote-reference/src/quantized.rs:177-201): 18 bytes = a little-endian
// binary16 scale d followed by 16 bytes; byte j holds element j in its low
// nibble and element j+16 in its high nibble, value (q - 8) * d.
//
// Two consecutive blocks ("a block pair", 36 bytes) start on a 4-byte boundary
// whenever the row and the matrix base do, so the kernels load a pair as nine
// dwords (dwordx4 + dwordx4 + dword) and never touch memory byte by byte.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "export.hpp"

namespace mote {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
// 16-byte vector that the compiler may only assume dword aligned.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr uint32_t kBlockElements = 32;
constexpr uint32_t kBlockBytes = 18;
constexpr uint32_t kPairBytes = 36;

// ---------------------------------------------------------------------------
// Nibble unpacking.
//
// A nibble n placed in mantissa bits [4, 8) of a binary16 whose exponent field
// encodes 2^0 (bits 0x3C00) is the exact value 1 + n/64.  One dword of four
// nibble bytes [b0 b1 b2 b3] therefore yields four packed f16 pairs with one
// AND-OR (plus a shift) each:
//   hi02 = ( q       & 0x00F000F0) | 0x3C003C00  -> (H(b0), H(b2))
//   lo02 = ((q << 4) & 0x00F000F0) | 0x3C003C00  -> (L(b0), L(b2))
//   lo13 = ((q >> 4) & 0x00F000F0) | 0x3C003C00  -> (L(b1), L(b3))
//   hi13 = ((q >> 8) & 0x00F000F0) | 0x3C003C00  -> (H(b1), H(b3))
// where L(bj) is element j (low nibble) and H(bj) element j+16 of the block.
// With acc = sum_k (1 + n_k/64) x_k accumulated by v_dot2_f32_f16 (the f16
// products are exact in f32),  sum_k (n_k - 8) x_k = 64 (acc - 1.125 sx)
// with sx = sum_k x_k over the block.
// ---------------------------------------------------------------------------
constexpr uint32_t kNibbleField = 0x00F000F0u;
constexpr uint32_t kOnePair = 0x3C003C00u;

__device__ __forceinline__ uint32_t nib_hi02(uint32_t q) { return (q & kNibbleField) | kOnePair; }
__device__ __forceinline__ uint32_t nib_lo02(uint32_t q) { return ((q << 4) & kNibbleField) | kOnePair; }
__device__ __forceinline__ uint32_t nib_lo13(uint32_t q) { return ((q >> 4) & kNibbleField) | kOnePair; }
__device__ __forceinline__ uint32_t nib_hi13(uint32_t q) { return ((q >> 8) & kNibbleField) | kOnePair; }

// The same with binary16 (1, 1) held in a VGPR (`one`, from one_pair_reg()):
// gfx9-family VOP3 instructions take no literal, so with the constant in a
// register each mask-and-insert is one v_and_or_b32 instead of an AND and an
// OR.  Bit-identical to the forms above.
__device__ __forceinline__ uint32_t one_pair_reg() {
    uint32_t one;
    asm("v_mov_b32 %0, 0x3c003c00" : "=v"(one));
    return one;
}
__device__ __forceinline__ uint32_t nib_hi02(uint32_t q, uint32_t one) { return (q & kNibbleField) | one; }
__device__ __forceinline__ uint32_t nib_lo02(uint32_t q, uint32_t one) { return ((q << 4) & kNibbleField) | one; }
__device__ __forceinline__ uint32_t nib_lo13(uint32_t q, uint32_t one) { return ((q >> 4) & kNibbleField) | one; }
__device__ __forceinline__ uint32_t nib_hi13(uint32_t q, uint32_t one) { return ((q >> 8) & kNibbleField) | one; }

__device__ __forceinline__ f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }

// v_dot2_f32_f16: a.lo*b.lo + a.hi*b.hi + c with f32 accumulation.
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

// Packs the binary16 halves x[a] (low) and x[b] (high) of a register array
// holding consecutive f16 pairs, with one v_perm_b32.
template <int A, int B>
__device__ __forceinline__ uint32_t pick_pair(const uint32_t* x) {
    constexpr uint32_t lo = (A & 1) ? 0x0302u : 0x0100u;          // bytes of S1
    constexpr uint32_t hi = (B & 1) ? 0x07060000u : 0x05040000u;  // bytes of S0
    return __builtin_amdgcn_perm(x[B / 2], x[A / 2], hi | lo);
}

__device__ __forceinline__ float half_lo_to_float(uint32_t v) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v & 0xffffu)));
}
__device__ __forceinline__ float half_hi_to_float(uint32_t v) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v >> 16)));
}

// Loads the nine dwords of the block pair that starts at `p` (4-byte aligned).
__device__ __forceinline__ void load_pair(const uint8_t* p, uint32_t (&d)[9]) {
    const u32x4_a4 a = *reinterpret_cast<const u32x4_a4*>(p);
    const u32x4_a4 b = *reinterpret_cast<const u32x4_a4*>(p + 16);
    const uint32_t c = *reinterpret_cast<const uint32_t*>(p + 32);
    d[0] = a.x; d[1] = a.y; d[2] = a.z; d[3] = a.w;
    d[4] = b.x; d[5] = b.y; d[6] = b.z; d[7] = b.w;
    d[8] = c;
}

// The eight nibble dwords of a pair in unpack order.  Block 0's nibble bytes
// sit at pair bytes 2..17, so its first dword is assembled from the high half
// of d0 (bytes 2,3 = elements 0,1) and the low half of d4 (bytes 16,17 =
// elements 14,15): byte order [e14 e15 e0 e1].  Block 1's nibbles are d5..d8.
__device__ __forceinline__ uint32_t pair_q0(const uint32_t (&d)[9]) {
    return __builtin_amdgcn_perm(d[0], d[4], 0x07060100u);  // (d4 & 0xFFFF) | (d0 & 0xFFFF0000)
}

// Block-local element index of byte position `pos` of nibble dword `w`
// (w = 0..3 block 0, 4..7 block 1) in the unpack order above.
__host__ __device__ constexpr int pair_byte_element(int w, int pos) {
    return (w == 0) ? (pos < 2 ? 14 + pos : pos - 2)
         : (w < 4)  ? (4 * w - 2 + pos)
                    : (4 * (w - 4) + pos);
}

// (q - 8) * d for the 8 nibbles of nibble dword q, in the order
// [b0.lo, b2.lo, b1.lo, b3.lo, b0.hi, b2.hi, b1.hi, b3.hi].  A low nibble
// masked into the mantissa of binary16 1024 (0x6400, ulp 1) reads 1024 + n; a
// high nibble left in place (bits 4-7) and masked into binary16 64 (0x5400,
// ulp 1/16) reads 64 + n, so one shift (by 8, for bytes 1 and 3) serves all
// four nibble pairs; adding -1032 or -72 gives n - 8 exactly and the multiply
// by d rounds once.  `c1024` and `c64` hold those constants in both halves in
// VGPRs: gfx9-family VOP3 instructions take no literal, so with the constant in
// a register each mask-and-insert is one v_and_or_b32 (mask in an SGPR).
__device__ __forceinline__ f16x8 dequant8(uint32_t q, f16x2 d, uint32_t c1024, uint32_t c64) {
    const f16x2 bias_lo = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
    const f16x2 bias_hi = {static_cast<_Float16>(-72.0f), static_cast<_Float16>(-72.0f)};
    const uint32_t q8 = q >> 8;
    const f16x2 l02 = (as_h2((q & 0x000F000Fu) | c1024) + bias_lo) * d;
    const f16x2 l13 = (as_h2((q8 & 0x000F000Fu) | c1024) + bias_lo) * d;
    const f16x2 h02 = (as_h2((q & 0x00F000F0u) | c64) + bias_hi) * d;
    const f16x2 h13 = (as_h2((q8 & 0x00F000F0u) | c64) + bias_hi) * d;
    return f16x8{l02.x, l02.y, l13.x, l13.y, h02.x, h02.y, h13.x, h13.y};
}

// GGML Q8_0 (crates/mote-reference/src/quantized.rs:191-195): a block is an
// f16 scale d and 32 two's-complement bytes v, value v d; a pair of blocks is
// 68 bytes (17 dwords), dword aligned whenever the row is.
constexpr uint32_t kQ8PairBytes = 68;

// Swizzled x stages in LDS: the 16-byte chunk 8 a + i of an activation row
// (bytes 16 i .. 16 i + 15 of its a-th 128) sits at position 8 a + ((i + a) &
// 7), so lanes reading their own 128 (or 64) contiguous bytes of x, chunk by
// chunk, spread over the banks instead of all hitting one bank row.
// swizzled_chunk(q): the chunk at position q; swizzled_position(c): the
// position of chunk c (its inverse).
__host__ __device__ constexpr uint32_t swizzled_chunk(uint32_t q) { return (q & ~7u) + (((q & 7u) - (q >> 3)) & 7u); }
__host__ __device__ constexpr uint32_t swizzled_position(uint32_t c) {
    return (c & ~7u) + (((c & 7u) + (c >> 3)) & 7u);
}

// Loads the seventeen dwords of the Q8_0 pair that starts at `p`.
__device__ __forceinline__ void load_pair_q8(const uint8_t* p, uint32_t (&d)[17]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const u32x4_a4 v = *reinterpret_cast<const u32x4_a4*>(p + 16 * i);
        d[4 * i + 0] = v.x; d[4 * i + 1] = v.y; d[4 * i + 2] = v.z; d[4 * i + 3] = v.w;
    }
    d[16] = *reinterpret_cast<const uint32_t*>(p + 64);
}

// Dword i (0..15) of a Q8_0 pair's 64 value bytes (elements 4i .. 4i + 3):
// block 0's bytes start at pair byte 2 and are re-aligned with one v_perm,
// block 1's are dwords 9 .. 16.
__device__ __forceinline__ uint32_t q8_bytes(const uint32_t (&d)[17], int i) {
    return i < 8 ? __builtin_amdgcn_perm(d[i + 1], d[i], 0x05040302u) : d[i + 1];
}

// Eight Q8_0 values (bytes b0..b3 of q0, b4..b7 of q1) times d, in the order
// [b0, b2, b1, b3, b4, b6, b5, b7], as a binary16 pair hi + lo: XOR 0x80 turns
// v into u = v + 128, a v_perm places u as the low byte of binary16 1024
// (0x64uu, ulp 1), which reads 1024 + u; adding -1152 gives v exactly; hi is
// v d rounded once and lo = fma(v, d, -hi) the rounded remainder, so hi + lo
// carries v d to about 2^-22 (a single binary16 product, enough for the
// 4-bit values of Q4_0, is not for 8-bit values).  `c64` holds 0x64 in every
// byte (a register: gfx9-family VOP3 instructions take no literal).
struct F16x8Pair {
    f16x8 hi, lo;
};
__device__ __forceinline__ F16x8Pair dequant8_q8(uint32_t q0, uint32_t q1, f16x2 d, uint32_t c64) {
    const f16x2 bias = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
    const uint32_t u0 = q0 ^ 0x80808080u, u1 = q1 ^ 0x80808080u;
    const f16x2 v02 = as_h2(__builtin_amdgcn_perm(c64, u0, 0x04020400u)) + bias;
    const f16x2 v13 = as_h2(__builtin_amdgcn_perm(c64, u0, 0x04030401u)) + bias;
    const f16x2 v46 = as_h2(__builtin_amdgcn_perm(c64, u1, 0x04020400u)) + bias;
    const f16x2 v57 = as_h2(__builtin_amdgcn_perm(c64, u1, 0x04030401u)) + bias;
    const f16x2 h02 = v02 * d, h13 = v13 * d, h46 = v46 * d, h57 = v57 * d;
    const f16x2 l02 = __builtin_elementwise_fma(v02, d, -h02), l13 = __builtin_elementwise_fma(v13, d, -h13);
    const f16x2 l46 = __builtin_elementwise_fma(v46, d, -h46), l57 = __builtin_elementwise_fma(v57, d, -h57);
    return {f16x8{h02.x, h02.y, h13.x, h13.y, h46.x, h46.y, h57.x, h57.y},
            f16x8{l02.x, l02.y, l13.x, l13.y, l46.x, l46.y, l57.x, l57.y}};
}

// ---------------------------------------------------------------------------
// Scales whose binary16 products overflow.
//
// The matrix-core kernels round each dequantised weight, (q - 8) d for Q4_0
// or v d for Q8_0, to binary16 before the MFMA.  With |q - 8| <= 8 the
// product stays finite for |d| <= 8188 (the largest binary16 below 8192); with
// |v| <= 128, for |d| <= 511.75.  The reference decodes in f32
// (crates/mote-reference/src/quantized.rs:187-195), where any finite d gives a
// finite value.  So when a wave's MFMA step holds a larger scale (no model's
// weights do), the step runs with every scale of the wave times 2^-S (S = 4
// for Q4_0, 8 for Q8_0, so 8 * 65504 / 16 and 128 * 65504 / 256 stay finite)
// and its f32 accumulators scaled by 2^-S before the step and by 2^S after.
// Scaling by a power of two is exact in f32, and in binary16 for every
// product that stays normal, so for Q4_0 the step computes exactly what an
// unbounded binary16 would wherever |d| >= 2^-10; scales below that in the
// same step as one of at least 8192, and the small low halves of Q8_0's
// hi + lo products, lose up to S bits to binary16 subnormals, which the
// tolerance, scaled by the largest |d|, absorbs by orders of magnitude.  Inf and NaN scales take the same path and propagate as the
// direct products would.  The test is one wave-uniform branch per step that
// ordinary weights never take; the step's code exists once, so the register
// use stays that of the ordinary step.
// ---------------------------------------------------------------------------
constexpr uint32_t kQ4BigScale = 0x7000u;  // binary16 8192: (q - 8) d may overflow from here
constexpr uint32_t kQ8BigScale = 0x6000u;  // binary16 512: v d may overflow from here
constexpr float kQ4BigDown = 0.0625f;      // 2^-4
constexpr float kQ8BigDown = 0.00390625f;  // 2^-8

// Whether either binary16 scale in the two halves of `scales` has a
// magnitude field of at least kLimit (inf and NaN included).
template <uint32_t kLimit>
__device__ __forceinline__ bool big_scales(uint32_t scales) {
    constexpr uint32_t kAdd = (0x8000u - kLimit) * 0x10001u;  // carries into bit 15 of a half from kLimit up
    return (((scales & 0x7FFF7FFFu) + kAdd) & 0x80008000u) != 0u;
}

__device__ __forceinline__ bool wave_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

// The two VGPR constants of dequant8.
struct DequantConsts {
    uint32_t c1024, c64, q8;  // q8: the 0x64 bytes of dequant8_q8
};
__device__ __forceinline__ DequantConsts dequant_consts() {
    DequantConsts c;
    asm("v_mov_b32 %0, 0x64006400" : "=v"(c.c1024));
    asm("v_mov_b32 %0, 0x54005400" : "=v"(c.c64));
    asm("v_mov_b32 %0, 0x64646464" : "=v"(c.q8));
    return c;
}

// ---------------------------------------------------------------------------
// Wave-level reduction with DPP (gfx9 row/bcast controls), result returned
// uniformly (read from lane 63).
// ---------------------------------------------------------------------------
template <int Ctrl, int RowMask = 0xF, int BankMask = 0xF, bool BoundCtrl = true>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
        0, __builtin_bit_cast(int, v), Ctrl, RowMask, BankMask, BoundCtrl));
}

__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<0xB1>(v);        // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);        // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);       // row_half_mirror
    v += dpp<0x140>(v);       // row_mirror: every lane of a row holds its row sum
    v += dpp<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3: lane 63 = total
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Output element conversion.
// SiLU of the fused gate/up epilogue, silu(g) = g / (1 + e^-g) in f32 with the
// device exponential, shared by every gate/up kernel so they agree bit for bit.
__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

template <typename T>
__device__ __forceinline__ T to_out(float v);
template <>
__device__ __forceinline__ float to_out<float>(float v) { return v; }
template <>
__device__ __forceinline__ _Float16 to_out<_Float16>(float v) { return static_cast<_Float16>(v); }

}  // namespace mote

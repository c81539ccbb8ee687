// K-quant super-block kernels for gfx950: Q4_K and Q6_K weights decoded to
// f32, and the weight-only linear y[M, N] = x[M, K] (f16) . W[N, K]^T for few
// tokens (the decode-shaped GEMV).
//
// The reference has the geometry of these formats only
// (crates/mote-types/src/lib.rs:39-74: 256 elements in 144 and 210 bytes, the
// "ggml-common.h ABI", storage alignment 4 and 2) and neither a kernel nor an
// oracle for them (crates/mote-reference/src/quantized.rs:154-156).  The
// layouts are GGML's block_q4_K and block_q6_K:
//
//  Q4_K, 144 bytes: f16 d, f16 dmin, scales[12], qs[128].  Element
//    64p + 32h + l (p = 0..3, h = 0..1, l = 0..31) is nibble h of qs[32p + l]
//    in sub-block j = 2p + h, value (d sc_j) q - dmin m_j, with the 6-bit sc_j
//    and m_j packed as: j < 4: sc = s[j] & 63, m = s[j + 4] & 63; j >= 4:
//    sc = (s[j + 4] & 15) | (s[j - 4] >> 6) << 4,
//    m = (s[j + 4] >> 4) | (s[j] >> 6) << 4.
//  Q6_K, 210 bytes: ql[128], qh[64], int8 scales[16], f16 d.  Element
//    128g + 32c + l (g = 0..1, c = 0..3, l = 0..31) is nibble (c >> 1) of
//    ql[64g + 32(c & 1) + l] with bits 2c..2c+1 of qh[32g + l] as bits 4..5,
//    value (d scales[e / 16]) (q - 32).
//
// Decode is bit-identical to the oracle: d sc and dmin m are exact in f32 (11
// + 6 significant bits), so is (d sc) q, and fma((d sc), q, -(dmin m)) is the
// one rounding of the exact Q4_K value that GGML's two f32 operations give;
// every Q6_K value (d sc)(q - 32) is exact (at most 23 significant bits).
//
// The linear (kq_gemv_kernel): workgroups of four waves, each wave owning R
// weight rows at a time and a token group of MT tokens (gridDim.y).  The
// activations of the token group are staged in LDS once per K chunk, in "pair
// order" (elements [a b c d] stored as [a c b d], so that the dword pairs
// (e, e + 2) and (e + 1, e + 3) line up with the nibble pairs one AND
// extracts), together with the f32 sum of every 16 consecutive activations.
// Eight lanes share a super-block, each taking 16 bytes of its quants (32
// elements, two scale groups), so a wave streams eight blocks of a row per
// step with 16-byte loads.  Quantized values enter v_dot2_f32_f16 as binary16
// subnormals (q 2^-24, or 2^-20 for the Q4_K high nibbles; products exact in
// f32, though the instruction's accumulation is not one IEEE rounding), and
// the per-group offsets (the Q4_K minimum, the Q6_K -32) are applied through
// the staged group sums:
//   Q4_K: sum_e x_e (d sc q_e - dmin m) = d sc 2^24 acc - dmin m S
//         (2^20 for the high nibbles' sums)
//   Q6_K: sum_e x_e d sc (q_e - 32)     = d sc (2^24 acc - 32 S).
// The LDS-ring GEMV (kq_ring_kernel) streams the same arithmetic for 1-4
// tokens per pass, and from 2 (Q4_K) or 5 (Q6_K) to 64 tokens at K <= 4096
// the matrix-core tiles (kq4_mfma_kernel, kq6_mfma_kernel) decode each block
// once per 16-token tile into exact binary16 operands.
// HBM-bound: algorithmic bytes per call are |W| + 2 M K + M N |y|.
#include "common.hpp"
#include "q4_0.hpp"

namespace mote::kquant {
namespace {

enum class Fmt { Q4K, Q6K };

constexpr uint32_t kSuper = 256;
constexpr int kGemvWaves = 4;
constexpr int kGemvThreads = kGemvWaves * kWave;
constexpr uint32_t kLdsBudget = 64 * 1024;  // x and group sums of one token group

template <Fmt F>
constexpr uint32_t block_bytes() {
    return F == Fmt::Q4K ? 144u : 210u;
}

__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}

// Sub-block j's 6-bit scale and min from the three dwords holding the 12
// scale bytes (s0 = s[0..3], s1 = s[4..7], s2 = s[8..11]).
__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t j, uint32_t& sc,
                                              uint32_t& m) {
    const uint32_t sh = 8u * (j & 3u);
    const uint32_t a = __builtin_amdgcn_ubfe(s0, sh, 8), b = __builtin_amdgcn_ubfe(s1, sh, 8);
    if (j < 4) {
        sc = a & 63u;
        m = b & 63u;
    } else {
        const uint32_t c = __builtin_amdgcn_ubfe(s2, sh, 8);
        sc = (c & 15u) | ((a >> 6) << 4);
        m = (c >> 4) | ((b >> 6) << 4);
    }
}

// 16 bytes at a 2-byte-aligned address, read as five dwords from the dword
// boundary at or below it; the caller guarantees the 20 bytes from there lie
// inside the object.
__device__ __forceinline__ u32x4 load16_a2(const uint8_t* p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t* q = reinterpret_cast<const uint32_t*>(a & ~uintptr_t{3});
    const uint32_t sh = static_cast<uint32_t>(a & 3u);  // 0 or 2
    const u32x4_a4 v = *reinterpret_cast<const u32x4_a4*>(q);
    const uint32_t e = q[4];
    u32x4 r;
    r.x = __builtin_amdgcn_alignbyte(v.y, v.x, sh);
    r.y = __builtin_amdgcn_alignbyte(v.z, v.y, sh);
    r.z = __builtin_amdgcn_alignbyte(v.w, v.z, sh);
    r.w = __builtin_amdgcn_alignbyte(e, v.w, sh);
    return r;
}

// ---------------------------------------------------------------------------
// Rows whose sum is not finite.  The linears below fold a sub-block's scale
// and min into sums over its elements (d sc sum x q - dmin m sum x); GGML's
// definition, which the oracle follows, rounds every element's value first
// (d1 = d sc, m1 = dmin m, then d1 q - m1 for Q4_K; (d sc)(q - 32) for
// Q6_K) and sums x times that.  With finite scales and activations neither
// form can overflow, so they agree to rounding; an infinite or NaN scale (or
// a non-finite activation) makes the folded sum not finite, and then it can
// put +-inf where the per-element values give NaN (inf * 0 for q = 0 or
// sc = 0, products of both signs).  A wave whose reduced sum is not finite (a
// wave-uniform test) recomputes its share of the row element by element, so
// the NaN and infinities land where the definition puts them.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool not_finite(float v) {
    return (__builtin_bit_cast(uint32_t, v) & 0x7F800000u) == 0x7F800000u;
}

// GGML's value of element e (0..255) of the super-block at `blk` (global
// memory), with the oracle's f32 rounding points.
template <Fmt F>
__device__ inline float kq_value(const uint8_t* blk, uint32_t e) {
    if constexpr (F == Fmt::Q4K) {
        const uint32_t p = e >> 6, h = (e >> 5) & 1u, l = e & 31u, j = 2 * p + h;
        const uint8_t* sb = blk + 4;
        uint32_t sc, m;
        if (j < 4) {
            sc = sb[j] & 63u;
            m = sb[j + 4] & 63u;
        } else {
            sc = (sb[j + 4] & 15u) | ((sb[j - 4] >> 6) << 4);
            m = (sb[j + 4] >> 4) | ((sb[j] >> 6) << 4);
        }
        const float d1 = half_bits_to_float(blk[0] | (blk[1] << 8)) * static_cast<float>(sc);
        const float m1 = half_bits_to_float(blk[2] | (blk[3] << 8)) * static_cast<float>(m);
        const uint32_t byte = blk[16 + 32 * p + l];
        const float prod = d1 * static_cast<float>(h ? byte >> 4 : byte & 15u);
        return prod - m1;
    } else {
        const uint32_t g = e >> 7, c = (e >> 5) & 3u, l = e & 31u;
        const uint32_t low = blk[64 * g + 32 * (c & 1u) + l] >> (4 * (c >> 1)) & 15u;
        const uint32_t high = (blk[128 + 32 * g + l] >> (2 * c)) & 3u;
        const float ds = half_bits_to_float(blk[208] | (blk[209] << 8)) *
                         static_cast<float>(static_cast<int8_t>(blk[192 + e / 16]));
        return ds * static_cast<float>(static_cast<int>(low | (high << 4)) - 32);
    }
}

// The wave's sum of x[k] * w[k] over blocks [b_begin, b_end) of the row at
// `row`, lanes over elements, with GGML's per-element values (rolled loop:
// it runs only for rows holding a non-finite scale or activation).
template <Fmt F>
__device__ inline float kq_exact_blocks(const uint8_t* row, const uint16_t* xrow, uint32_t b_begin, uint32_t b_end) {
    constexpr uint32_t BB = block_bytes<F>();
    float e = 0.0f;
    for (uint32_t k = b_begin * kSuper + (threadIdx.x & 63u); k < b_end * kSuper; k += 64u)
        e += half_bits_to_float(xrow[k]) * kq_value<F>(row + static_cast<size_t>(k / kSuper) * BB, k % kSuper);
    return wave_sum(e);
}

// ---------------------------------------------------------------------------
// Decode: one thread per 16 consecutive elements of a super-block.
// ---------------------------------------------------------------------------
template <bool VEC>
__device__ __forceinline__ void store16(float* out, const float (&v)[16]) {
    if constexpr (VEC) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            reinterpret_cast<f32x4*>(out)[i] = f32x4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) out[i] = v[i];
    }
}

template <bool VEC>
__global__ __launch_bounds__(256) void decode_q4k_kernel(const uint8_t* __restrict__ w, float* __restrict__ out,
                                                         uint64_t pieces) {
    const uint64_t t = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (t >= pieces) return;
    const uint64_t b = t >> 4;
    const uint32_t i = static_cast<uint32_t>(t & 15u);  // elements 16i .. 16i + 15
    const uint8_t* blk = w + b * 144;
    const u32x4_a4 hdr = *reinterpret_cast<const u32x4_a4*>(blk);
    const uint32_t p = i >> 2, h = (i >> 1) & 1u, l0 = 16u * (i & 1u);
    const u32x4_a4 qs = *reinterpret_cast<const u32x4_a4*>(blk + 16 + 32 * p + l0);
    uint32_t sc, m;
    q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * p + h, sc, m);
    const float d1 = half_bits_to_float(hdr.x & 0xffffu) * static_cast<float>(sc);
    const float m1 = half_bits_to_float(hdr.x >> 16) * static_cast<float>(m);
    const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
    float v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const uint32_t nib = (q[k >> 2] >> (8 * (k & 3) + 4 * h)) & 15u;
        v[k] = __builtin_fmaf(d1, static_cast<float>(nib), -m1);
    }
    store16<VEC>(out + t * 16, v);
}

template <bool VEC>
__global__ __launch_bounds__(256) void decode_q6k_kernel(const uint8_t* __restrict__ w, float* __restrict__ out,
                                                         uint64_t pieces) {
    const uint64_t t = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (t >= pieces) return;
    const uint64_t b = t >> 4;
    const uint32_t i = static_cast<uint32_t>(t & 15u);  // elements 16i .. 16i + 15
    const uint8_t* blk = w + b * 210;
    const uint32_t g = i >> 3, c = (i >> 1) & 3u, l0 = 16u * (i & 1u);
    const u32x4 ql = load16_a2(blk + 64 * g + 32 * (c & 1u) + l0);
    const u32x4 qh = load16_a2(blk + 128 + 32 * g + l0);
    const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(blk + 208));
    const float ds = d * static_cast<float>(static_cast<int8_t>(blk[192 + i]));
    const uint32_t lo[4] = {ql.x, ql.y, ql.z, ql.w}, hi[4] = {qh.x, qh.y, qh.z, qh.w};
    float v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const uint32_t sh = 8 * (k & 3);
        const uint32_t low = (lo[k >> 2] >> (sh + 4 * (c >> 1))) & 15u;
        const uint32_t high = (hi[k >> 2] >> (sh + 2 * c)) & 3u;
        v[k] = ds * static_cast<float>(static_cast<int>(low | (high << 4)) - 32);
    }
    store16<VEC>(out + t * 16, v);
}

// ---------------------------------------------------------------------------
// Linear.
// ---------------------------------------------------------------------------

// Stages tokens [0, mt) of the token group, elements [k0, k0 + kc), into LDS:
// xs[t][kc_max / 2] dwords in pair order and gs[t][kc_max / 16] group sums
// (kc <= kc_max, the row strides of the two arrays).
template <int MT>
__device__ __forceinline__ void stage_x(const uint16_t* __restrict__ x, uint32_t K, uint32_t k0, uint32_t kc,
                                        uint32_t kc_max, int mt, bool x16, uint32_t* xs, float* gs) {
    const uint32_t per_token = kc / 8;  // 8-element pieces (16 bytes) per token
    const uint32_t total = static_cast<uint32_t>(mt) * per_token;
    for (uint32_t idx = threadIdx.x; idx < total; idx += kGemvThreads) {
        const uint32_t t = idx / per_token, piece = idx - t * per_token;
        const uint16_t* src = x + static_cast<size_t>(t) * K + k0 + 8 * piece;
        uint32_t a[4];
        if (x16) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(src);
            a[0] = v.x; a[1] = v.y; a[2] = v.z; a[3] = v.w;
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = src[2 * i] | (static_cast<uint32_t>(src[2 * i + 1]) << 16);
        }
        // [x0 x1][x2 x3] -> [x0 x2][x1 x3]
        u32x4 o;
        o.x = __builtin_amdgcn_perm(a[1], a[0], 0x05040100u);
        o.y = __builtin_amdgcn_perm(a[1], a[0], 0x07060302u);
        o.z = __builtin_amdgcn_perm(a[3], a[2], 0x05040100u);
        o.w = __builtin_amdgcn_perm(a[3], a[2], 0x07060302u);
        *reinterpret_cast<u32x4*>(xs + t * (kc_max / 2) + 4 * piece) = o;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) s += half_bits_to_float(a[i] & 0xffffu) + half_bits_to_float(a[i] >> 16);
        // pieces 2q and 2q + 1 (adjacent lanes) form one 16-element group
        s += dpp<0xB1>(s);
        if ((piece & 1u) == 0) gs[t * (kc_max / 16) + piece / 2] = s;
    }
}

// One block's contribution for every token, lane part `part` (0..7).
template <Fmt F, int MT>
struct BlockPart;

template <int MT>
struct BlockPart<Fmt::Q4K, MT> {
    u32x4 hdr, qs;
    __device__ __forceinline__ void load(const uint8_t* blk, uint32_t part) {
        hdr = *reinterpret_cast<const u32x4_a4*>(blk);
        qs = *reinterpret_cast<const u32x4_a4*>(blk + 16 + 16 * part);
    }
    // e0: chunk-local element of the block's first element.
    __device__ __forceinline__ void accumulate(uint32_t part, uint32_t e0, int mt, const uint32_t* xs,
                                               const float* gs, uint32_t xs_stride, uint32_t gs_stride,
                                               float (&acc)[MT]) const {
        const uint32_t p = part >> 1, half = part & 1u;
        uint32_t sc0, m0, sc1, m1;
        q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * p, sc0, m0);
        q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * p + 1, sc1, m1);
        const float d = half_bits_to_float(hdr.x & 0xffffu), dmin = half_bits_to_float(hdr.x >> 16);
        // high nibbles masked in place (q & 0x00F000F0: n 2^-20, 16 times the
        // low nibbles' weight), so a1 carries 2^20 instead of 2^24
        const float a0 = d * static_cast<float>(sc0) * 16777216.0f, a1 = d * static_cast<float>(sc1) * 1048576.0f;
        const float c0 = dmin * static_cast<float>(m0), c1 = dmin * static_cast<float>(m1);
        const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
        uint32_t lo02[4], lo13[4], hi02[4], hi13[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t q8 = q[w] >> 8;
            lo02[w] = q[w] & 0x000F000Fu;
            lo13[w] = q8 & 0x000F000Fu;
            hi02[w] = q[w] & 0x00F000F0u;
            hi13[w] = q8 & 0x00F000F0u;
        }
        const uint32_t e_lo = e0 + 64 * p + 16 * half, e_hi = e_lo + 32;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m >= mt) break;
            const u32x4* xl = reinterpret_cast<const u32x4*>(xs + m * xs_stride + e_lo / 2);
            const u32x4* xh = reinterpret_cast<const u32x4*>(xs + m * xs_stride + e_hi / 2);
            const u32x4 l0 = xl[0], l1 = xl[1], h0 = xh[0], h1 = xh[1];
            const uint32_t xlo[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
            const uint32_t xhi[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
            float sl = 0.0f, sh = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                sl = dot2(lo02[w], xlo[2 * w], sl);
                sl = dot2(lo13[w], xlo[2 * w + 1], sl);
                sh = dot2(hi02[w], xhi[2 * w], sh);
                sh = dot2(hi13[w], xhi[2 * w + 1], sh);
            }
            const float g_lo = gs[m * gs_stride + e_lo / 16], g_hi = gs[m * gs_stride + e_hi / 16];
            float v = acc[m];
            v = __builtin_fmaf(a0, sl, v);
            v = __builtin_fmaf(-c0, g_lo, v);
            v = __builtin_fmaf(a1, sh, v);
            v = __builtin_fmaf(-c1, g_hi, v);
            acc[m] = v;
        }
    }
};

template <int MT>
struct BlockPart<Fmt::Q6K, MT> {
    u32x4 ql, qh;
    uint32_t d, s_lo, s_hi;
    __device__ __forceinline__ void load(const uint8_t* blk, uint32_t part) {
        const uint32_t g = part >> 2, c4 = part & 3u;
        ql = load16_a2(blk + 64 * g + 16 * c4);
        qh = load16_a2(blk + 128 + 32 * g + 16 * (c4 & 1u));
        s_lo = static_cast<uint32_t>(static_cast<int32_t>(static_cast<int8_t>(blk[192 + 8 * g + c4])));
        s_hi = static_cast<uint32_t>(static_cast<int32_t>(static_cast<int8_t>(blk[196 + 8 * g + c4])));
        d = *reinterpret_cast<const uint16_t*>(blk + 208);
    }
    __device__ __forceinline__ void accumulate(uint32_t part, uint32_t e0, int mt, const uint32_t* xs,
                                               const float* gs, uint32_t xs_stride, uint32_t gs_stride,
                                               float (&acc)[MT]) const {
        const uint32_t g = part >> 2, c4 = part & 3u;
        const uint32_t sh_lo = 2 * (c4 >> 1), sh_hi = 4 + 2 * (c4 >> 1);
        const float dd = half_bits_to_float(d);
        const float ds_lo = dd * static_cast<float>(static_cast<int32_t>(s_lo));
        const float ds_hi = dd * static_cast<float>(static_cast<int32_t>(s_hi));
        const float a_lo = ds_lo * 16777216.0f, a_hi = ds_hi * 16777216.0f;
        const float b_lo = ds_lo * 32.0f, b_hi = ds_hi * 32.0f;
        const uint32_t l[4] = {ql.x, ql.y, ql.z, ql.w}, h[4] = {qh.x, qh.y, qh.z, qh.w};
        uint32_t lo02[4], lo13[4], hi02[4], hi13[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t vlo = (l[w] & 0x0F0F0F0Fu) | (((h[w] >> sh_lo) & 0x03030303u) << 4);
            const uint32_t vhi = ((l[w] >> 4) & 0x0F0F0F0Fu) | (((h[w] >> sh_hi) & 0x03030303u) << 4);
            lo02[w] = vlo & 0x00FF00FFu;
            lo13[w] = (vlo >> 8) & 0x00FF00FFu;
            hi02[w] = vhi & 0x00FF00FFu;
            hi13[w] = (vhi >> 8) & 0x00FF00FFu;
        }
        const uint32_t e_lo = e0 + 128 * g + 16 * c4, e_hi = e_lo + 64;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m >= mt) break;
            const u32x4* xl = reinterpret_cast<const u32x4*>(xs + m * xs_stride + e_lo / 2);
            const u32x4* xh = reinterpret_cast<const u32x4*>(xs + m * xs_stride + e_hi / 2);
            const u32x4 l0 = xl[0], l1 = xl[1], h0 = xh[0], h1 = xh[1];
            const uint32_t xlo[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
            const uint32_t xhi[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
            float sl = 0.0f, sh = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                sl = dot2(lo02[w], xlo[2 * w], sl);
                sl = dot2(lo13[w], xlo[2 * w + 1], sl);
                sh = dot2(hi02[w], xhi[2 * w], sh);
                sh = dot2(hi13[w], xhi[2 * w + 1], sh);
            }
            const float g_lo = gs[m * gs_stride + e_lo / 16], g_hi = gs[m * gs_stride + e_hi / 16];
            float v = acc[m];
            v = __builtin_fmaf(a_lo, sl, v);
            v = __builtin_fmaf(-b_lo, g_lo, v);
            v = __builtin_fmaf(a_hi, sh, v);
            v = __builtin_fmaf(-b_hi, g_hi, v);
            acc[m] = v;
        }
    }
};

// kc: K chunk (a multiple of 256) whose activations fit the LDS budget.
template <Fmt F, int MT, int R, typename OutT>
__global__ __launch_bounds__(kGemvThreads) void kq_gemv_kernel(const uint16_t* __restrict__ x,
                                                              const uint8_t* __restrict__ w, OutT* __restrict__ y,
                                                              uint32_t M, uint32_t N, uint32_t K, uint32_t kc_max,
                                                              uint32_t x16) {
    extern __shared__ uint32_t lds[];
    uint32_t* xs = lds;
    float* gs = reinterpret_cast<float*>(lds + MT * (kc_max / 2));
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t part = lane & 7u, slot = lane >> 3;
    constexpr uint32_t BB = block_bytes<F>();
    const size_t row_bytes = static_cast<size_t>(K / kSuper) * BB;
    const uint32_t rows_per_group = kGemvWaves * R;
    const uint32_t groups = (N + rows_per_group - 1) / rows_per_group;
    const uint32_t chunks = (K + kc_max - 1) / kc_max;
    const uint32_t token_groups = (M + MT - 1) / MT;
    for (uint32_t tg = blockIdx.y; tg < token_groups; tg += gridDim.y) {
        const uint32_t m0 = tg * MT;
        const int mt = static_cast<int>(min(static_cast<uint32_t>(MT), M - m0));
        const uint16_t* xg = x + static_cast<size_t>(m0) * K;
        bool staged = false;
        for (uint32_t rg = blockIdx.x; rg < groups; rg += gridDim.x) {
            const uint32_t n0 = rg * rows_per_group + static_cast<uint32_t>(wave) * R;
            float acc[R][MT];
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;
            for (uint32_t c = 0; c < chunks; ++c) {
                const uint32_t k0 = c * kc_max, kc = min(kc_max, K - k0);
                if (chunks > 1 || !staged) {
                    __syncthreads();
                    stage_x<MT>(xg, K, k0, kc, kc_max, mt, x16 != 0, xs, gs);
                    __syncthreads();
                    staged = true;
                }
                const uint32_t nb = kc / kSuper;
                // Two block steps of all R rows are loaded before either is used.
                for (uint32_t jb = slot; jb < nb; jb += 16) {
                    const bool second = jb + 8 < nb;
                    BlockPart<F, MT> bp[2][R];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        if (n0 + r < N) {
                            const uint8_t* row =
                                w + static_cast<size_t>(n0 + r) * row_bytes + static_cast<size_t>(k0 / kSuper) * BB;
                            bp[0][r].load(row + static_cast<size_t>(jb) * BB, part);
                            if (second) bp[1][r].load(row + static_cast<size_t>(jb + 8) * BB, part);
                        }
                    }
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        if (n0 + r < N) {
                            bp[0][r].accumulate(part, jb * kSuper, mt, xs, gs, kc_max / 2, kc_max / 16, acc[r]);
                            if (second)
                                bp[1][r].accumulate(part, (jb + 8) * kSuper, mt, xs, gs, kc_max / 2, kc_max / 16,
                                                    acc[r]);
                        }
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (n0 + r >= N) continue;
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    if (m >= mt) break;
                    float s = wave_sum(acc[r][m]);
                    if (__builtin_expect(not_finite(s), 0))  // wave-uniform: the definition's per-element sum
                        s = kq_exact_blocks<F>(w + static_cast<size_t>(n0 + r) * row_bytes,
                                               x + static_cast<size_t>(m0 + m) * K, 0, K / kSuper);
                    if (lane == 0) y[static_cast<size_t>(m0 + m) * N + n0 + r] = to_out<OutT>(s);
                }
            }
        }
    }
}

int device_cus() {
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        return n;
    }();
    return cus;
}

constexpr int kRows = 2;

template <Fmt F, int MT, typename OutT>
hipError_t launch_gemv_mt(const void* x, const void* w, void* y, uint32_t M, uint32_t N, uint32_t K,
                          hipStream_t stream) {
    // the largest multiple of 256 whose activations and group sums, 2.25 MT
    // bytes per element, fit the budget
    uint32_t kc = kLdsBudget * 4 / (MT * 9) / kSuper * kSuper;
    if (kc > K) kc = K;
    const size_t lds = static_cast<size_t>(MT) * (kc / 2) * 4 + static_cast<size_t>(MT) * (kc / 16) * 4;
    const uint32_t groups = (N + kGemvWaves * kRows - 1) / (kGemvWaves * kRows);
    size_t fit = (160 * 1024) / (lds > 0 ? lds : 1);  // workgroups whose LDS fits one CU
    const uint32_t per_cu = static_cast<uint32_t>(fit < 1 ? 1 : (fit > 4 ? 4 : fit));
    uint32_t gx = K <= kc ? min(groups, static_cast<uint32_t>(device_cus()) * per_cu) : groups;
    if (gx == 0) gx = 1;
    const uint32_t token_groups = (M + MT - 1) / MT;
    const uint32_t gy = token_groups < 65535u ? token_groups : 65535u;
    const uint32_t x16 = (reinterpret_cast<uintptr_t>(x) & 15u) == 0 ? 1u : 0u;
    hipLaunchKernelGGL((kq_gemv_kernel<F, MT, kRows, OutT>), dim3(gx, gy), dim3(kGemvThreads), lds, stream,
                       static_cast<const uint16_t*>(x), static_cast<const uint8_t*>(w), static_cast<OutT*>(y), M, N,
                       K, kc, x16);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Few-token GEMV through per-wave LDS rings (kq_ring_kernel).
//
// One workgroup of eight waves per CU.  K is cut into S slices of at most 16
// super-blocks (S = 1, 2, 4 or 8; Q6_K slices are whole multiples of eight
// blocks so every slice starts on a 16-byte boundary); wave w takes slice
// w % S of row group w / S, so a workgroup computes 8 / S rows per step.
// Four lanes share a super-block, each with 64 elements of it: the lane's
// activations for those elements stay in registers for the whole kernel (32
// dwords per token in pair order, plus their group sums), and only weights
// stream.  A wave's slice of a row arrives in its LDS ring by coalesced
// non-temporal direct-to-LDS 16-byte loads (every lane of every load
// instruction active, chunk indexes clamped inside the slice, so each row
// issues exactly LOADS instructions and vmcnt counts rows), two rows ahead of
// the one computed and never past the wave's last row.  Lane j of a wave keeps the partial sum of step j % 64;
// every 64 steps the S partials of each row are added in slice order through
// LDS (bitwise reproducible) and stored.
//
// Requires: x and w 16-byte aligned, row bytes a multiple of 16 (Q6_K: K a
// multiple of 2048), K <= 32768.
// ---------------------------------------------------------------------------
constexpr int kRingWaves = 8;
constexpr int kRingThreads = kRingWaves * kWave;
constexpr int kRingSlots = 3;
typedef __attribute__((address_space(3))) void* lds_ptr;

// LDS store and load of one f32 that the compiler does not see as LDS
// accesses: with direct-to-LDS loads in flight, any LDS write it knows of
// makes it wait for all of them before every later LDS read.  Each completes
// before returning (lgkmcnt(0)).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr)(p)));
}
__device__ __forceinline__ void lds_store_f32_sync(uint32_t addr, float v) {
    asm volatile("ds_write_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" ::"v"(addr), "v"(v));
}
__device__ __forceinline__ float lds_load_f32_sync(uint32_t addr) {
    float r;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(r) : "v"(addr));
    return r;
}

template <Fmt F>
constexpr int ring_loads() {
    return F == Fmt::Q4K ? 3 : 4;  // 16 blocks = 144 / 210 chunks of 16 bytes
}

// The lane's activations: 64 elements of its block part for every token, in
// pair order, and the sums of its scale groups.
template <Fmt F, int MT>
struct LaneX {
    static constexpr int kGroups = F == Fmt::Q4K ? 2 : 4;
    uint32_t xr[MT][32];
    float sum[MT][kGroups];
};

// Element offsets (in the block) of the lane's two 32-element runs.
template <Fmt F>
__device__ __forceinline__ void part_runs(uint32_t part, uint32_t& e0, uint32_t& e1) {
    if constexpr (F == Fmt::Q4K) {
        e0 = 64 * part;
        e1 = e0 + 32;
    } else {
        e0 = 128 * (part >> 1) + 32 * (part & 1u);
        e1 = e0 + 64;
    }
}

// The lane's 64 activations of every token as loaded (two 32-element runs,
// 16 dwords each); issued before the first weight rows, used after them.
template <Fmt F, int MT>
__device__ __forceinline__ void load_lane_x(const uint16_t* __restrict__ x, uint32_t K, int mt, uint32_t elem0,
                                            uint32_t part, uint32_t (&raw)[MT][32]) {
    uint32_t e0, e1;
    part_runs<F>(part, e0, e1);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const int mm = m < mt ? m : mt - 1;  // tokens past the group re-read the last one
        const uint16_t* xr = x + static_cast<size_t>(mm) * K + elem0;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const u32x4* src = reinterpret_cast<const u32x4*>(xr + (r ? e1 : e0));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const u32x4 v = src[i];
                raw[m][16 * r + 4 * i + 0] = v.x; raw[m][16 * r + 4 * i + 1] = v.y;
                raw[m][16 * r + 4 * i + 2] = v.z; raw[m][16 * r + 4 * i + 3] = v.w;
            }
        }
    }
}

// Pair order and the group sums (32 elements for Q4_K, 16 for Q6_K).
template <Fmt F, int MT>
__device__ __forceinline__ void order_lane_x(const uint32_t (&raw)[MT][32], LaneX<F, MT>& lx) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            // [x0 x1][x2 x3] -> [x0 x2][x1 x3]
            lx.xr[m][2 * i] = __builtin_amdgcn_perm(raw[m][2 * i + 1], raw[m][2 * i], 0x05040100u);
            lx.xr[m][2 * i + 1] = __builtin_amdgcn_perm(raw[m][2 * i + 1], raw[m][2 * i], 0x07060302u);
        }
        constexpr int per = 32 / LaneX<F, MT>::kGroups;  // dwords of raw per group
#pragma unroll
        for (int g = 0; g < LaneX<F, MT>::kGroups; ++g) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < per; ++i) s = dot2(raw[m][g * per + i], kOnePair, s);
            lx.sum[m][g] = s;
        }
    }
}

// sum over the lane's 64 elements of x * w for every token, from the block at
// `blk` in LDS.
template <Fmt F, int MT>
__device__ __forceinline__ void ring_part_dot(uint32_t slot, uint32_t blk_off, uint32_t part,
                                              const LaneX<F, MT>& lx, float (&out)[MT]) {
    if constexpr (F == Fmt::Q4K) {
        // header, then the lane's 32 nibble bytes; LDS address `slot + blk_off`
        u32x4 hdr, qa, qb;
        const uint32_t ah = slot + blk_off, aq = ah + 16 + 32 * part;
        asm volatile(
            "ds_read_b128 %0, %3\n\t"
            "ds_read_b128 %1, %4\n\t"
            "ds_read_b128 %2, %4 offset:16\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(hdr), "=&v"(qa), "=&v"(qb)  // early clobber: no output may share an address register
            : "v"(ah), "v"(aq));
        uint32_t sc0, m0, sc1, m1;
        q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * part, sc0, m0);
        q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * part + 1, sc1, m1);
        const float d = half_bits_to_float(hdr.x & 0xffffu), dmin = half_bits_to_float(hdr.x >> 16);
        // high nibbles masked in place (n 2^-20), a1 scaled by 2^20: one shift
        // per dword instead of three.  Not bitwise the n 2^-24 form: measured
        // on MI355X, v_dot2_f32_f16 does not carry the smallest binary16
        // subnormals' products exactly, and this form is the closer to the f64
        // sums (largest error at 1 x 4096 x 4096 2.3e-4 against 4.3e-4)
        const float a0 = d * static_cast<float>(sc0) * 16777216.0f, a1 = d * static_cast<float>(sc1) * 1048576.0f;
        const float c0 = dmin * static_cast<float>(m0), c1 = dmin * static_cast<float>(m1);
        const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float lo = 0.0f, hi = 0.0f;
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                const uint32_t q8 = q[w] >> 8;
                lo = dot2(q[w] & 0x000F000Fu, lx.xr[m][2 * w], lo);
                lo = dot2(q8 & 0x000F000Fu, lx.xr[m][2 * w + 1], lo);
                hi = dot2(q[w] & 0x00F000F0u, lx.xr[m][16 + 2 * w], hi);
                hi = dot2(q8 & 0x00F000F0u, lx.xr[m][16 + 2 * w + 1], hi);
            }
            float v = a0 * lo;
            v = __builtin_fmaf(-c0, lx.sum[m][0], v);
            v = __builtin_fmaf(a1, hi, v);
            out[m] = __builtin_fmaf(-c1, lx.sum[m][1], v);
        }
    } else {
        const uint32_t g = part >> 1, c = part & 1u;
        // ql (32 bytes), qh (32 bytes) and the scale bytes 8g + 2c + {0, 1, 4, 5}
        // start at 2-byte offsets: each is read as dwords from the dword
        // boundary below it and realigned
        const uint32_t b = slot + blk_off;
        const uint32_t oq = b + 64 * g + 32 * c, oh = b + 128 + 32 * g, os = b + 192 + 8 * g + 2 * c;
        u32x2 l01, l23, l45, l67, h01, h23, h45, h67, s01;
        uint32_t l8, h8, s2, dbits;
        asm volatile(
            "ds_read2_b32 %0, %13 offset1:1\n\t"
            "ds_read2_b32 %1, %13 offset0:2 offset1:3\n\t"
            "ds_read2_b32 %2, %13 offset0:4 offset1:5\n\t"
            "ds_read2_b32 %3, %13 offset0:6 offset1:7\n\t"
            "ds_read_b32 %8, %13 offset:32\n\t"
            "ds_read2_b32 %4, %14 offset1:1\n\t"
            "ds_read2_b32 %5, %14 offset0:2 offset1:3\n\t"
            "ds_read2_b32 %6, %14 offset0:4 offset1:5\n\t"
            "ds_read2_b32 %7, %14 offset0:6 offset1:7\n\t"
            "ds_read_b32 %9, %14 offset:32\n\t"
            "ds_read2_b32 %10, %15 offset1:1\n\t"
            "ds_read_b32 %11, %15 offset:8\n\t"
            "ds_read_u16 %12, %16 offset:208\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(l01), "=&v"(l23), "=&v"(l45), "=&v"(l67), "=&v"(h01), "=&v"(h23), "=&v"(h45), "=&v"(h67),
              "=&v"(l8), "=&v"(h8), "=&v"(s01), "=&v"(s2), "=&v"(dbits)  // early clobber, as above
            : "v"(oq & ~3u), "v"(oh & ~3u), "v"(os & ~3u), "v"(b));
        const uint32_t lv[9] = {l01.x, l01.y, l23.x, l23.y, l45.x, l45.y, l67.x, l67.y, l8};
        const uint32_t hv[9] = {h01.x, h01.y, h23.x, h23.y, h45.x, h45.y, h67.x, h67.y, h8};
        const uint32_t sv[3] = {s01.x, s01.y, s2};
        uint32_t ql[8], qh[8], sc[2];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            ql[i] = __builtin_amdgcn_alignbyte(lv[i + 1], lv[i], oq & 2u);
            qh[i] = __builtin_amdgcn_alignbyte(hv[i + 1], hv[i], oh & 2u);
        }
        sc[0] = __builtin_amdgcn_alignbyte(sv[1], sv[0], os & 2u);
        sc[1] = __builtin_amdgcn_alignbyte(sv[2], sv[1], os & 2u);
        const float d = half_bits_to_float(dbits);
        // scales 8g + 2c + {0, 1} (low runs) in sc[0] bytes 0-1; 8g + 4 + 2c + {0, 1} in sc[1] bytes 0-1
        const float ds[4] = {
            d * static_cast<float>(static_cast<int8_t>(sc[0] & 0xffu)),
            d * static_cast<float>(static_cast<int8_t>((sc[0] >> 8) & 0xffu)),
            d * static_cast<float>(static_cast<int8_t>(sc[1] & 0xffu)),
            d * static_cast<float>(static_cast<int8_t>((sc[1] >> 8) & 0xffu)),
        };
        // The binary16-subnormal pairs straight from the bytes: quarter c's
        // q = nibble | 2 qh bits << 4 in bits 0-5 of each half (q 2^-24), and
        // quarter c + 2's in bits 4-9 (16 q 2^-24: its nibble masked in
        // place, its qh bits shifted to 8-9; 16 q <= 1008 stays subnormal), so
        // each pair is one mask and one v_and_or_b32 and the second quarter's
        // sums carry 2^20 instead of 2^24.  qh bits 2c, 2c + 1 (quarter c) and
        // 2c + 4, 2c + 5 (quarter c + 2) of bytes 0 and 2 reach bits 4-5 and
        // 8-9 shifted left by 4 - 2c; those of bytes 1 and 3 shifted right by
        // 4 + 2c.
        const uint32_t sh02 = 4 - 2 * c, sh13 = 4 + 2 * c;
        uint32_t v02[2][8], v13[2][8];
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const uint32_t l8 = ql[w] >> 8, h02 = qh[w] << sh02, h13 = qh[w] >> sh13;
            v02[0][w] = (ql[w] & 0x000F000Fu) | (h02 & 0x00300030u);
            v13[0][w] = (l8 & 0x000F000Fu) | (h13 & 0x00300030u);
            v02[1][w] = (ql[w] & 0x00F000F0u) | (h02 & 0x03000300u);
            v13[1][w] = (l8 & 0x00F000F0u) | (h13 & 0x03000300u);
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float v = 0.0f;
#pragma unroll
            for (int r = 0; r < 2; ++r) {
#pragma unroll
                for (int gi = 0; gi < 2; ++gi) {
                    float a = 0.0f;
#pragma unroll
                    for (int w = 4 * gi; w < 4 * gi + 4; ++w) {
                        a = dot2(v02[r][w], lx.xr[m][16 * r + 2 * w], a);
                        a = dot2(v13[r][w], lx.xr[m][16 * r + 2 * w + 1], a);
                    }
                    const float dsg = ds[2 * r + gi];
                    v = __builtin_fmaf(dsg * (r ? 1048576.0f : 16777216.0f), a, v);
                    v = __builtin_fmaf(-32.0f * dsg, lx.sum[m][2 * r + gi], v);
                }
            }
            out[m] = v;
        }
    }
}

// XL: the token group's activations are staged once per workgroup in LDS by
// direct-to-LDS loads (thread t loads 16-byte chunks t, t + 512, ... of each
// token, clamped, into 8 KB steps), issued before the first rows, and each
// lane reads its runs there after a barrier.  Without it every wave loads its
// lanes' activations from global memory: at one slice per row (K <= 4096 for
// Q4_K) the eight waves of a workgroup fetch the same x eight times.
template <Fmt F, int MT, int S, typename OutT, bool XL>
__global__ __launch_bounds__(kRingThreads) void kq_ring_kernel(const uint16_t* __restrict__ x,
                                                              const uint8_t* __restrict__ w, OutT* __restrict__ y,
                                                              uint32_t M, uint32_t N, uint32_t K, uint32_t slice_blocks) {
    constexpr int LOADS = ring_loads<F>();
    constexpr uint32_t kSlot = LOADS * 1024;
    constexpr uint32_t BB = block_bytes<F>();
    constexpr int RW = kRingWaves / S;
    __shared__ __attribute__((aligned(16))) uint8_t ring_lds[kRingWaves][kRingSlots][kSlot];
    __shared__ float part_lds[kRingWaves][kWave];
    extern __shared__ __attribute__((aligned(16))) uint8_t x_lds[];  // XL: [MT][ceil(K / 4096) 8 KB]
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t s = static_cast<uint32_t>(wave % S), rw = static_cast<uint32_t>(wave / S);
    const uint32_t nb = K / kSuper;
    const uint32_t b0 = min(s * slice_blocks, nb), b1 = min(b0 + slice_blocks, nb);
    // this wave's slice of a row in 16-byte chunks; an empty slice (possible
    // for the last Q6_K slices) loads the row's first chunk and drops it
    // (all its lanes are idle)
    const uint32_t chunks = b1 > b0 ? (b1 - b0) * BB / 16 : 1u;
    const size_t row_bytes = static_cast<size_t>(nb) * BB;
    const uint32_t blk = lane >> 2, part = lane & 3u;
    const bool active = b0 + blk < b1;
    const uint32_t keep = active ? 0xFFFFFFFFu : 0u;  // NaN-safe drop of idle lanes
    uint8_t* ring = &ring_lds[wave][0][0];
    const uint32_t row_steps = (N + RW - 1) / RW;

    for (uint32_t tg = blockIdx.y; tg * MT < M; tg += gridDim.y) {
        const uint32_t m0 = tg * MT;
        const int mt = static_cast<int>(min(static_cast<uint32_t>(MT), M - m0));
        const uint32_t steps = blockIdx.x < row_steps ? (row_steps - 1 - blockIdx.x) / gridDim.x + 1 : 0;
        auto row_of = [&](uint32_t t) { return (blockIdx.x + t * gridDim.x) * RW + rw; };
        auto load_row = [&](uint32_t t, uint32_t slot) {
            const uint32_t n = min(row_of(t), N - 1);  // past the end: re-read a row, never used
            const uint8_t* src = w + static_cast<size_t>(n) * row_bytes + static_cast<size_t>(b1 > b0 ? b0 : 0) * BB;
#pragma unroll
            for (int i = 0; i < LOADS; ++i) {
                const uint32_t c = min(64u * static_cast<uint32_t>(i) + lane, chunks - 1);
                __builtin_amdgcn_global_load_lds(src + 16u * c, (lds_ptr)(ring + slot * kSlot + 1024u * i), 16, 0,
                                                 2 /* non-temporal */);
            }
        };
        if (steps == 0) continue;  // uniform per workgroup
        __syncthreads();  // the previous token group's ring reads are done
        LaneX<F, MT> lx;
        if constexpr (XL) {
            const uint32_t xsteps = (K + 4095u) / 4096u, xstride = xsteps * 8192u;
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const int mm = m < mt ? m : mt - 1;  // tokens past the group re-read the last one
                const uint8_t* src = reinterpret_cast<const uint8_t*>(x + static_cast<size_t>(m0 + mm) * K);
                for (uint32_t i = 0; i < xsteps; ++i) {
                    // Q4_K: swizzled as the decode ring's x (chunk 8 a + i at 8 a + ((i + a) &
                    // 7)), since each lane reads 128 contiguous bytes below (1 x 4096 x 14336
                    // 8.36 -> 8.03 us, 1 x 4096 x 4096 4.92 -> 4.55); Q6_K's two 64-byte runs
                    // per lane measured level either way and stay unswizzled
                    const uint32_t q = 512u * i + threadIdx.x;
                    const uint32_t c = min(F == Fmt::Q4K ? swizzled_chunk(q) : q, K / 8u - 1u);
                    __builtin_amdgcn_global_load_lds(
                        src + 16u * c, (lds_ptr)(x_lds + m * xstride + 8192u * i + 1024u * static_cast<uint32_t>(wave)),
                        16, 0, 0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            load_row(0, 0);
            if (steps > 1) load_row(1, 1);
            __builtin_amdgcn_sched_barrier(0);
            // loads retire in order: with only the rows outstanding this
            // wave's x chunks have landed, and after the barrier every wave's
            if (steps > 1) __builtin_amdgcn_s_waitcnt(0x0F70 | (LOADS * 2));
            else __builtin_amdgcn_s_waitcnt(0x0F70 | LOADS);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            uint32_t raw[MT][32];
            uint32_t e0, e1;
            part_runs<F>(part, e0, e1);
            const uint32_t elem0 = min(b0 + blk, nb - 1) * kSuper;
#pragma unroll
            for (int m = 0; m < MT; ++m) {
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    const uint32_t c0 = (elem0 + (r ? e1 : e0)) / 8u;  // the run's first chunk
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t c = c0 + static_cast<uint32_t>(i);
                        const u32x4 v = *reinterpret_cast<const u32x4*>(
                            x_lds + m * xstride + 16u * (F == Fmt::Q4K ? swizzled_position(c) : c));
                        raw[m][16 * r + 4 * i + 0] = v.x; raw[m][16 * r + 4 * i + 1] = v.y;
                        raw[m][16 * r + 4 * i + 2] = v.z; raw[m][16 * r + 4 * i + 3] = v.w;
                    }
                }
            }
            order_lane_x<F, MT>(raw, lx);
        } else {
            uint32_t raw[MT][32];
            load_lane_x<F, MT>(x + static_cast<size_t>(m0) * K, K, mt, min(b0 + blk, nb - 1) * kSuper, part, raw);
            __builtin_amdgcn_sched_barrier(0);
            load_row(0, 0);
            if (steps > 1) load_row(1, 1);
            __builtin_amdgcn_sched_barrier(0);
            order_lane_x<F, MT>(raw, lx);
        }
        float mine[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) mine[m] = 0.0f;
        for (uint32_t t = 0; t < steps; ++t) {
            // Rows are loaded only up to the last step, so the count of loads
            // still allowed in flight once row t has landed shrinks at the end.
            if (t + 2 < steps) {
                load_row(t + 2, (t + 2) % kRingSlots);
                __builtin_amdgcn_s_waitcnt(0x0F70 | (LOADS * 2));
            } else if (t + 1 < steps) {
                __builtin_amdgcn_s_waitcnt(0x0F70 | LOADS);
            } else {
                __builtin_amdgcn_s_waitcnt(0x0F70);
            }
            __builtin_amdgcn_sched_barrier(0);
            float part_sum[MT];
            ring_part_dot<F, MT>(lds_addr(ring + (t % kRingSlots) * kSlot), blk * BB, part, lx, part_sum);
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const float v = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, part_sum[m]) & keep);
                float tot = wave_sum(v);
                if (__builtin_expect(not_finite(tot), 0)) {  // wave-uniform: the definition's per-element sum
                    const int mm = m < mt ? m : mt - 1;
                    tot = kq_exact_blocks<F>(w + static_cast<size_t>(min(row_of(t), N - 1)) * row_bytes,
                                             x + static_cast<size_t>(m0 + mm) * K, b0, b1);
                }
                mine[m] = lane == (t & 63u) ? tot : mine[m];
            }
            if ((t & 63u) == 63u || t + 1 == steps) {
                const uint32_t first = t & ~63u, count = (t & 63u) + 1;
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    if (m >= mt) break;
                    float total = mine[m];
                    if constexpr (S > 1) {
                        lds_store_f32_sync(lds_addr(&part_lds[wave][lane]), mine[m]);
                        __builtin_amdgcn_s_barrier();
                        total = 0.0f;
#pragma unroll
                        for (int k = 0; k < S; ++k) total += lds_load_f32_sync(lds_addr(&part_lds[rw * S + k][lane]));
                        __builtin_amdgcn_s_barrier();
                    }
                    const uint32_t n = row_of(first + lane);
                    if (s == 0 && lane < count && n < N) y[static_cast<size_t>(m0 + m) * N + n] = to_out<OutT>(total);
                }
            }
        }
    }
}

template <Fmt F>
bool ring_supported(const void* x, const void* w, uint32_t K) {
    const uint32_t nb = K / kSuper;
    if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0 || (reinterpret_cast<uintptr_t>(w) & 15u) != 0) return false;
    if (nb == 0 || nb > 128) return false;
    return F == Fmt::Q4K || nb % 8 == 0;
}

template <Fmt F, int MT, int S, typename OutT>
hipError_t launch_ring_s(const void* x, const void* w, void* y, uint32_t M, uint32_t N, uint32_t K,
                         uint32_t slice_blocks, hipStream_t stream) {
    constexpr uint32_t RW = kRingWaves / S;
    const uint32_t row_steps = (N + RW - 1) / RW;
    uint32_t gx = static_cast<uint32_t>(device_cus());
    if (gx > row_steps) gx = row_steps;
    const uint32_t groups = (M + MT - 1) / MT;
    const uint32_t gy = groups < 65535u ? groups : 65535u;
    // Q4_K: x through LDS where several row groups share a slice and the
    // staged tokens fit beside the rings (static: rings and partial sums).
    // Measured on MI355X: 1 x 4096 x 14336 9.05 -> 8.53 us, 2 tokens 12.23
    // -> 11.10, 8 tokens 33.2 -> 30.4, 14336 x 4096 10.35 -> 9.86.  Q6_K keeps
    // the per-wave loads: staged, its 2-8 token passes ran 3-5 % slower
    // (4 x 4096 x 14336: 19.2 against 18.7 us) and one token gained 0-2 %.
    constexpr size_t kStatic = sizeof(uint8_t) * kRingWaves * kRingSlots * ring_loads<F>() * 1024 +
                               sizeof(float) * kRingWaves * kWave;
    const size_t xl = static_cast<size_t>(MT) * ((K + 4095u) / 4096u) * 8192u;
    const auto* xp = static_cast<const uint16_t*>(x);
    const auto* wp = static_cast<const uint8_t*>(w);
    auto* yp = static_cast<OutT*>(y);
    if (F == Fmt::Q4K && RW > 1 && kStatic + xl <= 160u * 1024u)
        hipLaunchKernelGGL((kq_ring_kernel<F, MT, S, OutT, true>), dim3(gx, gy), dim3(kRingThreads), xl, stream, xp,
                           wp, yp, M, N, K, slice_blocks);
    else
        hipLaunchKernelGGL((kq_ring_kernel<F, MT, S, OutT, false>), dim3(gx, gy), dim3(kRingThreads), 0, stream, xp,
                           wp, yp, M, N, K, slice_blocks);
    return hipGetLastError();
}

template <Fmt F, int MT, typename OutT>
hipError_t launch_ring_mt(const void* x, const void* w, void* y, uint32_t M, uint32_t N, uint32_t K,
                          hipStream_t stream) {
    const uint32_t nb = K / kSuper;
    uint32_t S = 1;
    while ((nb + S - 1) / S > 16) S *= 2;
    uint32_t sb = (nb + S - 1) / S;
    if (F == Fmt::Q6K) sb = (sb + 7) / 8 * 8;
    switch (S) {
        case 1: return launch_ring_s<F, MT, 1, OutT>(x, w, y, M, N, K, sb, stream);
        case 2: return launch_ring_s<F, MT, 2, OutT>(x, w, y, M, N, K, sb, stream);
        case 4: return launch_ring_s<F, MT, 4, OutT>(x, w, y, M, N, K, sb, stream);
        default: return launch_ring_s<F, MT, 8, OutT>(x, w, y, M, N, K, sb, stream);
    }
}

// ---------------------------------------------------------------------------
// Q4_K on the matrix cores (kq4_mfma_kernel): 2 to 64 tokens, K parts of up
// to KS x STEPS super-blocks (4096).
//
// v_mfma_f32_16x16x32_f16 with the activations as the A operand (16 tokens)
// and the weights as the B operand (16 rows), so the lane that holds output
// (token, row) is one of the four lanes that loaded that row's block header:
// d, dmin and the sub-block scales stay in the lane.  Wave kw of a workgroup
// owns super-blocks kw, kw + KS, ... of every row and keeps the activations of
// those blocks for the workgroup's 16-token tile in registers; lane group g
// takes bytes qs[32 g .. 32 g + 31] of a block, i.e. sub-blocks 2 g (low
// nibbles) and 2 g + 1 (high nibbles), 64 elements.  MFMA t (of 8 per block)
// takes 8 of them: nibble h = t / 4 of bytes 8 (t % 4) .. 8 (t % 4) + 7.  The
// weight operand is sc_j q, exact in binary16 (at most 63 x 15): q enters as
// 1024 + q (low nibble masked into binary16 1024) or 64 + q (high nibble into
// binary16 64, ulp 1/16), and one packed fma with (sc, -1024 sc) or
// (sc, -64 sc) gives sc q exactly.  Each product with an activation is exact
// in f32, so one f32 accumulator per block holds sum_j sc_j sum x q; the
// minimum term sum_j m_j S_tj (S_tj: token t's sum over sub-block j) is a
// second MFMA pair with S split into binary16 hi + lo (m exact), and
//   y[t, r] += d_r C[t, r] - dmin_r C'[t, r]
// once per block in f32.  GGML's definition rounds each element's value
// (d1 q - m1) instead; the difference is rounding only.  The KS waves' partial
// tiles meet in LDS and are summed in wave order (deterministic).  A result
// that is not finite (an infinite or NaN scale, a non-finite activation) is
// recomputed by its thread element by element with the definition's values,
// so NaN and infinities land where the oracle puts them.  Split K (K past
// 4096): each workgroup keeps one K part of 16 super-blocks and writes that
// part's f32 plane of the partial tiles (recomputing a non-finite part over
// the part's elements); kq_splitk_reduce_kernel adds the planes in part order.
// ---------------------------------------------------------------------------

// sum over the row of x[k] w[k] with GGML's per-element values, one thread.
template <Fmt F>
__device__ inline float kq_exact_thread(const uint8_t* row, const uint16_t* xrow, uint32_t nb) {
    float acc = 0.0f;
    for (uint32_t k = 0; k < nb * kSuper; ++k)
        acc += half_bits_to_float(xrow[k]) *
               kq_value<F>(row + static_cast<size_t>(k / kSuper) * block_bytes<F>(), k % kSuper);
    return acc;
}

__device__ __forceinline__ uint32_t kq_pick(const uint32_t* x, int a, int b) {
    const uint32_t lo = (a & 1) ? 0x0302u : 0x0100u;
    const uint32_t hi = (b & 1) ? 0x07060000u : 0x05040000u;
    return __builtin_amdgcn_perm(x[b >> 1], x[a >> 1], hi | lo);
}

__device__ __forceinline__ uint32_t f16x2_bits(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }

// Activations of one super-block (512 bytes per token) for the 16 tokens of a
// token tile, loaded whole cache lines per instruction and handed out through
// a wave-private LDS region.  Load instruction c covers tokens 2c and 2c + 1
// (lanes 0-31 and 32-63, 16 bytes each), so each instruction reads 8 whole
// 128-byte lines once; loaded per lane instead (each lane its own 128 bytes of
// one token), every instruction touched 64 lines and the 16 waves' lines
// outgrew the vector L1, which fetched them again.  Round r then passes tokens
// 4r .. 4r + 3 through the region: every lane writes what it loaded for them,
// and the lanes of those tokens (li = token) read the eight 16-byte chunks at
// byte offsets off(0..7) of their token's slice (a wave's LDS operations
// complete in order).  Tokens past M read row M - 1 (lines the wave already
// holds in L1; loads skipped per instruction compiled to a chain of waits):
// a token only feeds its own output row of the MFMA, and those rows are never
// stored.  Rounds whose tokens all lie past M are skipped (uniform), and the
// lanes of such tokens keep zeros.
constexpr int kXRowBytes = 512 + 16;  // a token's slice plus padding, per LDS row
constexpr int kXRoundTokens = 4;
constexpr int kXStageBytes = kXRoundTokens * kXRowBytes;  // per wave

template <typename Off>
__device__ __forceinline__ void stage_block_x(const uint16_t* __restrict__ x, uint32_t K, uint32_t M, uint32_t tok0,
                                              uint32_t b, int lane, uint8_t* xs, Off off, uint32_t (&xr)[32]) {
    const int li = lane & 15;
    u32x4 g[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const uint32_t m = min(tok0 + 2u * c + static_cast<uint32_t>(lane >> 5), M - 1);
        g[c] = *reinterpret_cast<const u32x4*>(x + static_cast<size_t>(m) * K + static_cast<size_t>(b) * kSuper +
                                               static_cast<uint32_t>(lane & 31) * 8u);
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) xr[i] = 0u;
#pragma unroll
    for (int r = 0; r < 16 / kXRoundTokens; ++r) {
        if (tok0 + static_cast<uint32_t>(r * kXRoundTokens) < M) {  // uniform
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int tr = 2 * j + (lane >> 5);  // token within the round
                *reinterpret_cast<u32x4*>(xs + tr * kXRowBytes + (lane & 31) * 16) = g[2 * r + j];
            }
            if (li / kXRoundTokens == r) {
                const uint8_t* row = xs + (li % kXRoundTokens) * kXRowBytes;
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const u32x4 v = *reinterpret_cast<const u32x4*>(row + off(c));
                    xr[4 * c] = v.x; xr[4 * c + 1] = v.y; xr[4 * c + 2] = v.z; xr[4 * c + 3] = v.w;
                }
            }
        }
    }
}

template <int KS, int STEPS, typename OutT, bool SK = false>
__global__ __launch_bounds__(KS * 64) void kq4_mfma_kernel(const uint16_t* __restrict__ x, const uint8_t* __restrict__ w,
                                                          OutT* __restrict__ y, uint32_t M, uint32_t N, uint32_t K,
                                                          uint32_t token_tiles, uint32_t items, uint32_t per_xcd,
                                                          uint32_t kparts, float* __restrict__ partial) {
    constexpr int kLazy = KS * 64 / 256;  // items reduced together: one output per thread
    __shared__ float part[kLazy][KS][16][17];  // [item][wave][token][row]
    __shared__ __attribute__((aligned(16))) uint8_t xstage[KS][kXStageBytes];
    const int tid = static_cast<int>(threadIdx.x);
    const int kw = tid >> 6, lane = tid & 63, li = lane & 15, lg = lane >> 4;
    const uint32_t nb = K / kSuper;
    const size_t row_bytes = static_cast<size_t>(nb) * 144;
    const uint32_t groups = gridDim.x;
    // XCD-aware order: workgroups of one XCD take consecutive items, so the
    // token tiles of a row tile read its weights through the same L2.  Items
    // are (row tile, token tile, K part); the grid is a multiple of the
    // combos, so a workgroup keeps one token tile and one K part (SK: KS x
    // STEPS super-blocks from b0; without split K, all of K).
    const uint32_t first = (blockIdx.x % 8u) * per_xcd + blockIdx.x / 8u;
    const uint32_t combos = SK ? token_tiles * kparts : token_tiles;
    const uint32_t tok0 = (first % token_tiles) * 16u;
    const uint32_t b0 = SK ? (first % combos) / token_tiles * (KS * STEPS) : 0u;

    // The activations of this wave's blocks for the 16 tokens: the MFMA
    // operands (permuted to the weight operands' element order) and the
    // sub-block sums as binary16 hi + lo pairs.  Tokens past M stay zero.
    uint32_t xa[STEPS][8][4];
    uint32_t s_hi[STEPS], s_lo[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
        const uint32_t b = b0 + static_cast<uint32_t>(kw) + KS * static_cast<uint32_t>(s);
        uint32_t xr[32];
        if (b < nb) {  // uniform
            // lane (li, lg): elements 64 lg .. 64 lg + 63 of token li
            stage_block_x(x, K, M, tok0, b, lane, xstage[kw], [&](int c) { return 128 * lg + 16 * c; }, xr);
        } else {
#pragma unroll
            for (int i = 0; i < 32; ++i) xr[i] = 0u;
        }
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            s0 = dot2(xr[i], kOnePair, s0);
            s1 = dot2(xr[16 + i], kOnePair, s1);
        }
        const _Float16 h0 = static_cast<_Float16>(s0), h1 = static_cast<_Float16>(s1);
        const _Float16 l0 = static_cast<_Float16>(s0 - static_cast<float>(h0));
        const _Float16 l1 = static_cast<_Float16>(s1 - static_cast<float>(h1));
        s_hi[s] = f16x2_bits(f16x2{h0, h1});
        s_lo[s] = f16x2_bits(f16x2{l0, l1});
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int e = 32 * (t >> 2) + 8 * (t & 3);
            xa[s][t][0] = kq_pick(xr, e, e + 2);
            xa[s][t][1] = kq_pick(xr, e + 1, e + 3);
            xa[s][t][2] = kq_pick(xr, e + 4, e + 6);
            xa[s][t][3] = kq_pick(xr, e + 5, e + 7);
        }
    }

    // binary16 1024 and 64 in both halves of a VGPR, so that each
    // mask-and-insert below is one v_and_or_b32 (a VOP3 takes no literal)
    const DequantConsts dq = dequant_consts();

    // This lane's part of a row's block: the 16-byte header (d, dmin, the 12
    // scale bytes) and its 32 nibble bytes.
    struct Part {
        u32x4 hdr, qa, qb;
    };
    auto load_part = [&](uint32_t item, int s, Part& pt) {
        const uint32_t b = b0 + static_cast<uint32_t>(kw) + KS * static_cast<uint32_t>(s);
        if (b >= nb) return;  // uniform: a step past the row's blocks
        const uint32_t n = min((item / combos) * 16u + static_cast<uint32_t>(li), N - 1);
        const uint8_t* base = w + static_cast<size_t>(n) * row_bytes + static_cast<size_t>(b) * 144;
        pt.hdr = *reinterpret_cast<const u32x4*>(base);
        pt.qa = *reinterpret_cast<const u32x4*>(base + 16 + 32 * lg);
        pt.qb = *reinterpret_cast<const u32x4*>(base + 32 + 32 * lg);
    };
    // One block of one item: sum_j sc_j q x on the matrix cores, the minimum
    // term, and y += d C - dmin C' for this lane's four (token, row) outputs.
    auto block_mfma = [&](const Part& pt, int s, f32x4 yv) {
        uint32_t sc0, m0, sc1, m1;
        q4k_scale_min(pt.hdr.y, pt.hdr.z, pt.hdr.w, 2u * lg, sc0, m0);
        q4k_scale_min(pt.hdr.y, pt.hdr.z, pt.hdr.w, 2u * lg + 1u, sc1, m1);
        const _Float16 f0 = static_cast<_Float16>(static_cast<float>(sc0));
        const _Float16 f1 = static_cast<_Float16>(static_cast<float>(sc1));
        const f16x2 sc_lo = {f0, f0}, sc_hi = {f1, f1};
        const f16x2 b_lo = {static_cast<_Float16>(-1024.0f * static_cast<float>(sc0)),
                            static_cast<_Float16>(-1024.0f * static_cast<float>(sc0))};
        const f16x2 b_hi = {static_cast<_Float16>(-64.0f * static_cast<float>(sc1)),
                            static_cast<_Float16>(-64.0f * static_cast<float>(sc1))};
        const uint32_t q[8] = {pt.qa.x, pt.qa.y, pt.qa.z, pt.qa.w, pt.qb.x, pt.qb.y, pt.qb.z, pt.qb.w};
        f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t qa = q[2 * (t & 3)], qb = q[2 * (t & 3) + 1];
            f16x2 v[4];
            if (t < 4) {  // low nibbles: 1024 + q, then sc q
                v[0] = as_h2((qa & 0x000F000Fu) | dq.c1024);
                v[1] = as_h2(((qa >> 8) & 0x000F000Fu) | dq.c1024);
                v[2] = as_h2((qb & 0x000F000Fu) | dq.c1024);
                v[3] = as_h2(((qb >> 8) & 0x000F000Fu) | dq.c1024);
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = __builtin_elementwise_fma(v[i], sc_lo, b_lo);
            } else {  // high nibbles: 64 + q, then sc q
                v[0] = as_h2((qa & 0x00F000F0u) | dq.c64);
                v[1] = as_h2(((qa >> 8) & 0x00F000F0u) | dq.c64);
                v[2] = as_h2((qb & 0x00F000F0u) | dq.c64);
                v[3] = as_h2(((qb >> 8) & 0x00F000F0u) | dq.c64);
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = __builtin_elementwise_fma(v[i], sc_hi, b_hi);
            }
            const f16x8 bw = {v[0].x, v[0].y, v[1].x, v[1].y, v[2].x, v[2].y, v[3].x, v[3].y};
            const f16x8 ax = __builtin_bit_cast(f16x8, u32x4{xa[s][t][0], xa[s][t][1], xa[s][t][2], xa[s][t][3]});
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax, bw, c, 0, 0, 0);
        }
        // sum_j m_j S_tj: k slots 8 g and 8 g + 1 hold sub-blocks 2 g, 2 g + 1
        const uint32_t mw = f16x2_bits(f16x2{static_cast<_Float16>(static_cast<float>(m0)),
                                              static_cast<_Float16>(static_cast<float>(m1))});
        const f16x8 bm = __builtin_bit_cast(f16x8, u32x4{mw, 0u, 0u, 0u});
        f32x4 cm = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, u32x4{s_hi[s], 0u, 0u, 0u}), bm,
                                                          f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
        cm = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, u32x4{s_lo[s], 0u, 0u, 0u}), bm, cm, 0, 0,
                                                    0);
        const float d = half_bits_to_float(pt.hdr.x & 0xffffu), dmin = half_bits_to_float(pt.hdr.x >> 16);
#pragma unroll
        for (int r = 0; r < 4; ++r) yv[r] = __builtin_fmaf(-dmin, cm[r], __builtin_fmaf(d, c[r], yv[r]));
        return yv;
    };
    Part cur[STEPS];
    if (first < items) {
#pragma unroll
        for (int s = 0; s < STEPS; ++s) load_part(first, s, cur[s]);
    }
    // Items of this workgroup in chunks of kLazy: each wave streams its block
    // of every item of the chunk with the next item's loads in flight and
    // keeps the partial tiles in registers; the chunk's tiles then meet in
    // LDS behind one barrier (instead of two barriers per item).
    for (uint32_t c0 = first; c0 < items; c0 += kLazy * groups) {  // uniform per workgroup
        f32x4 yacc[kLazy];
#pragma unroll
        for (int i = 0; i < kLazy; ++i) {
            yacc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            const uint32_t item = c0 + static_cast<uint32_t>(i) * groups;
            if (item >= items) break;  // uniform
            const uint32_t next = item + groups;
#pragma unroll
            for (int s = 0; s < STEPS; ++s) {
                const uint32_t b = b0 + static_cast<uint32_t>(kw) + KS * static_cast<uint32_t>(s);
                if (b < nb) {  // uniform
                    const Part pt = cur[s];
                    if (next < items) load_part(next, s, cur[s]);  // the next item's block under this one's MFMAs
                    yacc[i] = block_mfma(pt, s, yacc[i]);
                }
            }
        }
        // lane holds tokens 4 g .. 4 g + 3 of row li of each item; the KS
        // partial tiles meet in LDS and are summed in wave order
#pragma unroll
        for (int i = 0; i < kLazy; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) part[i][kw][4 * lg + r][li] = yacc[i][r];
        __syncthreads();
        {
            const int i = tid >> 8, tok = (tid >> 4) & 15, row = tid & 15;  // KS * 64 >= kLazy * 256 threads
            const uint32_t item = c0 + static_cast<uint32_t>(i) * groups;
            const uint32_t m = tok0 + static_cast<uint32_t>(tok);
            const uint32_t n = (item / combos) * 16u + static_cast<uint32_t>(row);
            if (i < kLazy && item < items && m < M && n < N) {
                float v = part[i][0][tok][row];
#pragma unroll
                for (int k = 1; k < KS; ++k) v += part[i][k][tok][row];
                // not finite: the definition's per-element sum over this K part
                if (__builtin_expect(not_finite(v), 0))
                    v = kq_exact_thread<Fmt::Q4K>(w + static_cast<size_t>(n) * row_bytes + static_cast<size_t>(b0) * 144,
                                                  x + static_cast<size_t>(m) * K + static_cast<size_t>(b0) * kSuper,
                                                  SK ? min(static_cast<uint32_t>(KS * STEPS), nb - b0) : nb);
                if constexpr (SK)  // this K part's plane of the partial sums
                    partial[(static_cast<size_t>(b0 / (KS * STEPS)) * M + m) * N + n] = v;
                else
                    y[static_cast<size_t>(m) * N + n] = to_out<OutT>(v);
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Q6_K on the matrix cores (kq6_mfma_kernel), 5 to 64 tokens, K parts of up
// to KS super-blocks (4096):
// the Q4_K tile's layout (16 tokens as the A operand, 16 weight rows as the B
// operand, one super-block per wave, partial tiles summed in LDS in wave
// order).
//
// Lane group g takes ql bytes 32 g .. 32 g + 31: half p = g / 2 of the block
// and quarters c = g % 2 (low nibbles) and g % 2 + 2 (high nibbles), i.e.
// elements 128 p + 32 c + l, l = 0..31, with the qh bytes 32 p + l.  MFMA
// t = 4 h + u takes l = 8 u .. 8 u + 7 of quarter c = g % 2 + 2 h, eight
// elements of one 16-element sub-block (scale 8 p + 2 c + u / 2), in their
// natural order, so the activations enter the A operand as they lie in
// memory.  The 6-bit q (nibble | two qh bits << 4) enters binary16 as
// 1024 + q (one v_perm with 0x64 high bytes), and the weight operand
// sc (q - 32) is split over two MFMAs: sc = 8 s + t with s = sc >> 3 in
// [-16, 15] and t = sc & 7, so (q - 32) s (at most 512) and (q - 32) t (at
// most 224) are exact binary16 integers, each one packed fma from 1024 + q,
// and every product with an activation is exact in f32.  Per block
//   y[t, r] += d_r (8 C_s[t, r] + C_t[t, r]).
// GGML's definition rounds each element's value (d sc)(q - 32) (exact) and
// sums x times it; the difference is rounding only.  A result that is not
// finite is recomputed by its thread element by element, as in the Q4_K tile.
// Blocks lie at 2-byte offsets (210-byte blocks).  Where a row is a whole
// number of 16-byte units (K a multiple of 2048: A16), block b of every row
// sits 2 (b mod 8) bytes past a 16-byte boundary -- the same offset for all
// lanes of the wave that owns it -- so each 32-byte run is read as three
// aligned 16-byte chunks and realigned by that wave-uniform offset (the chunks
// end at most 2 bytes before the block's end).  Otherwise each 16 bytes are
// read as five dwords from the dword boundary at or below them.  Either way
// every read stays inside the block or the one before it (w is 16-byte
// aligned).  The four scales come as one 8-byte read from the dword boundary
// at or below them, d as a 16-bit word.
// ---------------------------------------------------------------------------

// The 32 bytes at p, p = 16 a + 4 o4 + sh (o4 and sh the same in every lane),
// from the three 16-byte chunks at 16 a.
__device__ __forceinline__ void load32_u(const uint8_t* p, uint32_t o4, uint32_t sh, u32x4& lo, u32x4& hi) {
    const u32x4* q = reinterpret_cast<const u32x4*>(reinterpret_cast<uintptr_t>(p) & ~uintptr_t{15});
    const u32x4 a = q[0], b = q[1], c = q[2];
    const uint32_t d[12] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c.x, c.y, c.z, c.w};
    uint32_t o[8];
    switch (o4) {  // uniform
#define MOTE_Q6_REALIGN(S)                                                                      \
    case S:                                                                                     \
        for (int k = 0; k < 8; ++k) o[k] = __builtin_amdgcn_alignbyte(d[k + S + 1], d[k + S], sh); \
        break;
        MOTE_Q6_REALIGN(0)
        MOTE_Q6_REALIGN(1)
        MOTE_Q6_REALIGN(2)
        default:
        MOTE_Q6_REALIGN(3)
#undef MOTE_Q6_REALIGN
    }
    lo = u32x4{o[0], o[1], o[2], o[3]};
    hi = u32x4{o[4], o[5], o[6], o[7]};
}

template <int KS, bool A16, typename OutT, bool SK = false>
__global__ __launch_bounds__(KS * 64) void kq6_mfma_kernel(const uint16_t* __restrict__ x, const uint8_t* __restrict__ w,
                                                          OutT* __restrict__ y, uint32_t M, uint32_t N, uint32_t K,
                                                          uint32_t token_tiles, uint32_t items, uint32_t per_xcd,
                                                          uint32_t kparts, float* __restrict__ partial) {
    constexpr int kLazy = KS * 64 / 256;  // items reduced together: one output per thread
    __shared__ float part[kLazy][KS][16][17];  // [item][wave][token][row]
    __shared__ __attribute__((aligned(16))) uint8_t xstage[KS][kXStageBytes];
    const int tid = static_cast<int>(threadIdx.x);
    const int kw = tid >> 6, lane = tid & 63, li = lane & 15, lg = lane >> 4;
    const uint32_t half = static_cast<uint32_t>(lg) >> 1, c0 = static_cast<uint32_t>(lg) & 1u;
    const uint32_t nb = K / kSuper;
    const size_t row_bytes = static_cast<size_t>(nb) * 210;
    const uint32_t groups = gridDim.x;
    // items and K parts as in the Q4_K tile (SK: KS super-blocks from b0)
    const uint32_t first = (blockIdx.x % 8u) * per_xcd + blockIdx.x / 8u;
    const uint32_t combos = SK ? token_tiles * kparts : token_tiles;
    const uint32_t tok0 = (first % token_tiles) * 16u;
    const uint32_t b0 = SK ? (first % combos) / token_tiles * KS : 0u;
    const uint32_t b = b0 + static_cast<uint32_t>(kw);  // this wave's super-block

    // The activations of this wave's block for the 16 tokens: quarter c0 + 2 h,
    // elements 8 u .. 8 u + 7 in xa[4 h + u] (byte 256 half + 64 c0 + 128 h +
    // 16 u of the token's slice).
    uint32_t xa[8][4];
    {
        uint32_t xr[32];
        if (b < nb) {  // uniform
            stage_block_x(x, K, M, tok0, b, lane, xstage[kw],
                          [&](int t) { return 256 * half + 64 * c0 + 128 * (t >> 2) + 16 * (t & 3); }, xr);
        } else {
#pragma unroll
            for (int i = 0; i < 32; ++i) xr[i] = 0u;
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            xa[t][0] = xr[4 * t]; xa[t][1] = xr[4 * t + 1]; xa[t][2] = xr[4 * t + 2]; xa[t][3] = xr[4 * t + 3];
        }
    }

    // This lane's part of a row's block: 32 ql bytes, the 32 qh bytes of its
    // half, the scales of its four sub-blocks (two 16-bit words) and d.
    struct Part {
        u32x4 l0, l1, h0, h1;
        uint32_t s_lo, s_hi, d;
    };
    auto load_part = [&](uint32_t item, Part& pt) {
        if (b >= nb) return;  // uniform: a wave past the row's blocks
        const uint32_t n = min((item / combos) * 16u + static_cast<uint32_t>(li), N - 1);
        const uint8_t* base = w + static_cast<size_t>(n) * row_bytes + static_cast<size_t>(b) * 210;
        if constexpr (A16) {
            const uint32_t o = 2u * (b & 7u);  // base mod 16
            load32_u(base + 32 * lg, (o + 32u * lg) % 16u / 4u, o & 3u, pt.l0, pt.l1);
            load32_u(base + 128 + 32 * half, o / 4u, o & 3u, pt.h0, pt.h1);
        } else {
            pt.l0 = load16_a2(base + 32 * lg);
            pt.l1 = load16_a2(base + 32 * lg + 16);
            pt.h0 = load16_a2(base + 128 + 32 * half);
            pt.h1 = load16_a2(base + 128 + 32 * half + 16);
        }
        // scale bytes s = 192 + 8 half + 2 c0 (+1) and s + 4 (+1): one 8-byte
        // read from the dword boundary at or below s (s - 2 >= 190, s + 6 <= 208)
        const uint8_t* sp = base + 192 + 8 * half + 2 * c0;
        const uint32_t ssh = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sp) & 3u);  // 0 or 2
        typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));
        const u32x2_a4 sv = *reinterpret_cast<const u32x2_a4*>(reinterpret_cast<uintptr_t>(sp) & ~uintptr_t{3});
        pt.s_lo = __builtin_amdgcn_alignbyte(sv.y, sv.x, ssh) & 0xFFFFu;
        pt.s_hi = (ssh ? sv.y >> 16 : sv.y) & 0xFFFFu;
        pt.d = *reinterpret_cast<const uint16_t*>(base + 208);
    };
    const uint32_t sh_lo = 4u - 2u * c0, sh_hi = 2u * c0;  // qh bits 2c..2c+1 to bits 4..5
    auto block_mfma = [&](const Part& pt, f32x4 yv) {
        const uint32_t L[8] = {pt.l0.x, pt.l0.y, pt.l0.z, pt.l0.w, pt.l1.x, pt.l1.y, pt.l1.z, pt.l1.w};
        const uint32_t H[8] = {pt.h0.x, pt.h0.y, pt.h0.z, pt.h0.w, pt.h1.x, pt.h1.y, pt.h1.z, pt.h1.w};
        f32x4 cs = {0.0f, 0.0f, 0.0f, 0.0f}, ct = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {  // sub-block j of this quarter: u = 2 j, 2 j + 1
                const int sc = static_cast<int8_t>(((h ? pt.s_hi : pt.s_lo) >> (8 * j)) & 0xFFu);
                const _Float16 fs = static_cast<_Float16>(static_cast<float>(sc >> 3));
                const _Float16 ft = static_cast<_Float16>(static_cast<float>(sc & 7));
                const _Float16 gs = static_cast<_Float16>(-1056.0f * static_cast<float>(sc >> 3));
                const _Float16 gt = static_cast<_Float16>(-1056.0f * static_cast<float>(sc & 7));
                const f16x2 ms = {fs, fs}, as = {gs, gs}, mt = {ft, ft}, at = {gt, gt};
#pragma unroll
                for (int uu = 0; uu < 2; ++uu) {
                    const int u = 2 * j + uu;
                    uint32_t q[2];
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        const uint32_t l = L[2 * u + i], hb = H[2 * u + i];
                        q[i] = h == 0 ? (l & 0x0F0F0F0Fu) | ((hb << sh_lo) & 0x30303030u)
                                      : ((l >> 4) & 0x0F0F0F0Fu) | ((hb >> sh_hi) & 0x30303030u);
                    }
                    f16x2 v[4];  // 1024 + q, elements 8 u .. 8 u + 7 in order
                    v[0] = as_h2(__builtin_amdgcn_perm(0x64646464u, q[0], 0x04010400u));
                    v[1] = as_h2(__builtin_amdgcn_perm(0x64646464u, q[0], 0x04030402u));
                    v[2] = as_h2(__builtin_amdgcn_perm(0x64646464u, q[1], 0x04010400u));
                    v[3] = as_h2(__builtin_amdgcn_perm(0x64646464u, q[1], 0x04030402u));
                    f16x2 vs[4], vt[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        vs[i] = __builtin_elementwise_fma(v[i], ms, as);  // (q - 32) s
                        vt[i] = __builtin_elementwise_fma(v[i], mt, at);  // (q - 32) t
                    }
                    const f16x8 ax =
                        __builtin_bit_cast(f16x8, u32x4{xa[4 * h + u][0], xa[4 * h + u][1], xa[4 * h + u][2], xa[4 * h + u][3]});
                    const f16x8 bs = {vs[0].x, vs[0].y, vs[1].x, vs[1].y, vs[2].x, vs[2].y, vs[3].x, vs[3].y};
                    const f16x8 bt = {vt[0].x, vt[0].y, vt[1].x, vt[1].y, vt[2].x, vt[2].y, vt[3].x, vt[3].y};
                    cs = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax, bs, cs, 0, 0, 0);
                    ct = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax, bt, ct, 0, 0, 0);
                }
            }
        }
        const float d = half_bits_to_float(pt.d);
#pragma unroll
        for (int r = 0; r < 4; ++r) yv[r] = __builtin_fmaf(d, __builtin_fmaf(8.0f, cs[r], ct[r]), yv[r]);
        return yv;
    };
    Part cur;
    if (first < items) load_part(first, cur);
    for (uint32_t c0i = first; c0i < items; c0i += kLazy * groups) {  // uniform per workgroup
        // each item's partial tile goes to LDS as soon as it is formed
#pragma unroll
        for (int i = 0; i < kLazy; ++i) {
            const uint32_t item = c0i + static_cast<uint32_t>(i) * groups;
            if (item >= items) break;  // uniform
            const uint32_t next = item + groups;
            f32x4 yv = {0.0f, 0.0f, 0.0f, 0.0f};
            if (b < nb) {  // uniform
                const Part pt = cur;
                if (next < items) load_part(next, cur);  // the next item's block under this one's MFMAs
                yv = block_mfma(pt, yv);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) part[i][kw][4 * lg + r][li] = yv[r];
        }
        __syncthreads();
        {
            const int i = tid >> 8, tok = (tid >> 4) & 15, row = tid & 15;
            const uint32_t item = c0i + static_cast<uint32_t>(i) * groups;
            const uint32_t m = tok0 + static_cast<uint32_t>(tok);
            const uint32_t n = (item / combos) * 16u + static_cast<uint32_t>(row);
            if (i < kLazy && item < items && m < M && n < N) {
                float v = part[i][0][tok][row];
#pragma unroll
                for (int k = 1; k < KS; ++k) v += part[i][k][tok][row];
                // not finite: the definition's per-element sum over this K part
                if (__builtin_expect(not_finite(v), 0))
                    v = kq_exact_thread<Fmt::Q6K>(w + static_cast<size_t>(n) * row_bytes + static_cast<size_t>(b0) * 210,
                                                  x + static_cast<size_t>(m) * K + static_cast<size_t>(b0) * kSuper,
                                                  SK ? min(static_cast<uint32_t>(KS), nb - b0) : nb);
                if constexpr (SK)  // this K part's plane of the partial sums
                    partial[(static_cast<size_t>(b0 / KS) * M + m) * N + n] = v;
                else
                    y[static_cast<size_t>(m) * N + n] = to_out<OutT>(v);
            }
        }
        __syncthreads();
    }
}

// The matrix-core tiles: 16-token tiles, one workgroup of 16 waves per CU,
// one block per wave: K <= 4096 in one pass (a Q4_K wave's activations for
// more blocks outgrow its registers: 16 waves of two blocks, or 8 of four,
// spill), longer K in parts of 16 super-blocks whose partial tiles a second
// kernel adds in part order (split K; the last part may be short); x and w
// 16-byte aligned.  From 2 tokens for Q4_K in one pass (2 x 4096 x 14336:
// 10.5 us on the tile, 11.1 on the ring), 3 with split K (2 x 14336 x 4096:
// 13.2 us on the tiles and the part sum, 12.8 on the ring; 3 tokens: 13.3
// against 21.0), and 5 for Q6_K: below that the ring GEMV's single pass of up
// to four tokens is faster (3 / 4 x 4096 x 14336: 18.9 / 19.2 us on the ring,
// 19.7 on the tile; 4 x 14336 x 4096: 20.6 on the ring, 22.5 on the split
// tiles at 5 tokens).
template <Fmt F>
bool kq_mfma_supported(const void* x, const void* w, uint32_t M, uint32_t K) {
    const uint32_t nb = K / kSuper;
    const uint32_t min_m = F == Fmt::Q4K ? (nb <= 16 ? 2u : 3u) : 5u;
    return M >= min_m && M <= 64 && nb >= 1 &&
           (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<uintptr_t>(w) & 15u) == 0;
}

// y[i] = the sum of the K parts' planes at i, in part order, converted.
template <typename OutT>
__global__ __launch_bounds__(256) void kq_splitk_reduce_kernel(const float* __restrict__ partial, uint32_t kparts,
                                                               uint64_t count, OutT* __restrict__ y) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x; i < count;
         i += static_cast<uint64_t>(gridDim.x) * 256) {
        float v = partial[i];
        for (uint32_t k = 1; k < kparts; ++k) v += partial[static_cast<uint64_t>(k) * count + i];
        y[i] = to_out<OutT>(v);
    }
}

// Returns hipErrorStreamCaptureUnsupported, with nothing queued, when split K
// needs more scratch than a stream under graph capture holds (the caller then
// runs the ring GEMV).
template <Fmt F, typename OutT>
hipError_t launch_kq_mfma(const void* x, const void* w, void* y, uint32_t M, uint32_t N, uint32_t K,
                          hipStream_t stream) {
    constexpr int KS = 16;
    const uint32_t nb = K / kSuper;
    const uint32_t kparts = (nb + KS - 1) / KS;
    const uint32_t token_tiles = (M + 15) / 16;
    const uint32_t row_tiles = (N + 15) / 16;
    const uint64_t items64 = static_cast<uint64_t>(row_tiles) * token_tiles * kparts;
    if (items64 > 0x7fffffffull) return hipErrorInvalidConfiguration;
    const uint32_t items = static_cast<uint32_t>(items64);
    // whole XCD rounds that are also a multiple of the (token tile, K part)
    // combos, so every workgroup keeps one token tile and K part
    const uint32_t combos = token_tiles * kparts;
    uint32_t a = 8u, b = combos;
    while (b != 0) { const uint32_t t = a % b; a = b; b = t; }
    const uint32_t unit = 8u / a * combos;
    uint32_t groups = static_cast<uint32_t>(device_cus());
    if (groups > items) groups = items;
    groups = (groups + unit - 1) / unit * unit;
    const auto* xp = static_cast<const uint16_t*>(x);
    const auto* wp = static_cast<const uint8_t*>(w);
    auto* yp = static_cast<OutT*>(y);
    if (kparts == 1) {
        if constexpr (F == Fmt::Q4K)
            hipLaunchKernelGGL((kq4_mfma_kernel<KS, 1, OutT>), dim3(groups), dim3(KS * 64), 0, stream, xp, wp, yp, M, N,
                               K, token_tiles, items, groups / 8u, 1u, nullptr);
        else if (K % 2048 == 0)
            hipLaunchKernelGGL((kq6_mfma_kernel<KS, true, OutT>), dim3(groups), dim3(KS * 64), 0, stream, xp, wp, yp, M,
                               N, K, token_tiles, items, groups / 8u, 1u, nullptr);
        else
            hipLaunchKernelGGL((kq6_mfma_kernel<KS, false, OutT>), dim3(groups), dim3(KS * 64), 0, stream, xp, wp, yp,
                               M, N, K, token_tiles, items, groups / 8u, 1u, nullptr);
        return hipGetLastError();
    }
    // Split K: the stream's scratch is held until both kernels are queued
    // (the lease goes out of scope at return).  Its layout is the Q4_0 split
    // K's: the tile arrival counters first (cleared when the buffer is new,
    // since the Q4_0 folded epilogue expects them zero), then the partial
    // tiles, [kparts][M][N] f32.
    const uint64_t count = static_cast<uint64_t>(M) * N;
    q4_0::ScratchPool::Lease lease;
    const hipError_t se =
        q4_0::acquire_scratch(stream, q4_0::kSplitKCounterBytes + count * kparts * sizeof(float), &lease);
    if (se != hipSuccess) return se;
    auto* base = static_cast<uint8_t*>(lease.ptr());
    if (lease.fresh()) {
        const hipError_t z = q4_0::launch_zero_fill(base, q4_0::kSplitKCounterBytes / 4, q4_0::OutType::F32, stream);
        if (z != hipSuccess) return z;
    }
    auto* part = reinterpret_cast<float*>(base + q4_0::kSplitKCounterBytes);
    if constexpr (F == Fmt::Q4K)
        hipLaunchKernelGGL((kq4_mfma_kernel<KS, 1, OutT, true>), dim3(groups), dim3(KS * 64), 0, stream, xp, wp, yp, M,
                           N, K, token_tiles, items, groups / 8u, kparts, part);
    else if (K % 2048 == 0)
        hipLaunchKernelGGL((kq6_mfma_kernel<KS, true, OutT, true>), dim3(groups), dim3(KS * 64), 0, stream, xp, wp, yp,
                           M, N, K, token_tiles, items, groups / 8u, kparts, part);
    else
        hipLaunchKernelGGL((kq6_mfma_kernel<KS, false, OutT, true>), dim3(groups), dim3(KS * 64), 0, stream, xp, wp,
                           yp, M, N, K, token_tiles, items, groups / 8u, kparts, part);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const uint64_t blocks = (count + 255) / 256;
    hipLaunchKernelGGL((kq_splitk_reduce_kernel<OutT>), dim3(static_cast<uint32_t>(blocks < 2048 ? blocks : 2048)),
                       dim3(256), 0, stream, part, kparts, count, yp);
    return hipGetLastError();
}

template <Fmt F, typename OutT>
hipError_t launch_gemv(const void* x, const void* w, void* y, uint32_t M, uint32_t N, uint32_t K,
                       hipStream_t stream) {
    if (kq_mfma_supported<F>(x, w, M, K)) {
        const hipError_t e = launch_kq_mfma<F, OutT>(x, w, y, M, N, K, stream);
        if (e != hipErrorStreamCaptureUnsupported) return e;  // else: split K under capture without scratch
    }
    if (ring_supported<F>(x, w, K)) {
        if (M == 1) return launch_ring_mt<F, 1, OutT>(x, w, y, M, N, K, stream);
        if (M == 2) return launch_ring_mt<F, 2, OutT>(x, w, y, M, N, K, stream);
        return launch_ring_mt<F, 4, OutT>(x, w, y, M, N, K, stream);
    }
    if (M == 1) return launch_gemv_mt<F, 1, OutT>(x, w, y, M, N, K, stream);
    if (M == 2) return launch_gemv_mt<F, 2, OutT>(x, w, y, M, N, K, stream);
    if (M <= 4) return launch_gemv_mt<F, 4, OutT>(x, w, y, M, N, K, stream);
    return launch_gemv_mt<F, 8, OutT>(x, w, y, M, N, K, stream);
}

template <Fmt F>
int linear(const void* input, const void* weights, void* output, uint64_t rows, uint64_t n, uint64_t k,
           bool f16_out, void* stream) {
    if (!input || !weights || !output || !stream) return hipErrorInvalidValue;
    if (k % kSuper != 0) return hipErrorInvalidValue;
    const uintptr_t walign = F == Fmt::Q4K ? 4 : 2;
    if ((reinterpret_cast<uintptr_t>(weights) & (walign - 1)) != 0 || (reinterpret_cast<uintptr_t>(input) & 1u) != 0 ||
        (reinterpret_cast<uintptr_t>(output) & (f16_out ? 1u : 3u)) != 0)
        return hipErrorInvalidValue;
    if (rows == 0 || n == 0) return hipSuccess;
    if (rows > UINT_MAX || n > UINT_MAX || rows > UINT_MAX / n) return hipErrorInvalidConfiguration;
    if (k > 0x7fffffffull) return hipErrorInvalidConfiguration;
    const auto s = static_cast<hipStream_t>(stream);
    if (k == 0)
        return static_cast<int>(q4_0::launch_zero_fill(output, rows * n, f16_out ? q4_0::OutType::F16 : q4_0::OutType::F32, s));
    const auto M = static_cast<uint32_t>(rows), N = static_cast<uint32_t>(n), K = static_cast<uint32_t>(k);
    const hipError_t e = f16_out ? launch_gemv<F, _Float16>(input, weights, output, M, N, K, s)
                                 : launch_gemv<F, float>(input, weights, output, M, N, K, s);
    return static_cast<int>(e);
}

template <Fmt F>
int dequantize(const void* weights, void* output, uint64_t rows, uint64_t k, void* stream) {
    if (!weights || !output || !stream) return hipErrorInvalidValue;
    if (k % kSuper != 0) return hipErrorInvalidValue;
    const uintptr_t walign = F == Fmt::Q4K ? 4 : 2;
    if ((reinterpret_cast<uintptr_t>(weights) & (walign - 1)) != 0 || (reinterpret_cast<uintptr_t>(output) & 3u) != 0)
        return hipErrorInvalidValue;
    if (rows == 0 || k == 0) return hipSuccess;
    if (rows > (1ull << 40) / k) return hipErrorInvalidConfiguration;
    const uint64_t pieces = rows * (k / 16);
    const uint64_t grid = (pieces + 255) / 256;
    if (grid > 0x7fffffffull) return hipErrorInvalidConfiguration;
    const bool vec = (reinterpret_cast<uintptr_t>(output) & 15u) == 0;
    const auto s = static_cast<hipStream_t>(stream);
    const auto* wp = static_cast<const uint8_t*>(weights);
    auto* op = static_cast<float*>(output);
    if constexpr (F == Fmt::Q4K) {
        if (vec)
            hipLaunchKernelGGL(decode_q4k_kernel<true>, dim3(static_cast<uint32_t>(grid)), dim3(256), 0, s, wp, op, pieces);
        else
            hipLaunchKernelGGL(decode_q4k_kernel<false>, dim3(static_cast<uint32_t>(grid)), dim3(256), 0, s, wp, op, pieces);
    } else {
        if (vec)
            hipLaunchKernelGGL(decode_q6k_kernel<true>, dim3(static_cast<uint32_t>(grid)), dim3(256), 0, s, wp, op, pieces);
        else
            hipLaunchKernelGGL(decode_q6k_kernel<false>, dim3(static_cast<uint32_t>(grid)), dim3(256), 0, s, wp, op, pieces);
    }
    return static_cast<int>(hipGetLastError());
}

}  // namespace
}  // namespace mote::kquant

using mote::kquant::Fmt;

MOTE_EXPORT int mote_hip_quantized_linear_q4_k_f32(const void* input, const void* weights, void* output,
                                                  uint64_t rows, uint64_t output_features,
                                                  uint64_t input_features, void* stream) noexcept {
    return mote::kquant::linear<Fmt::Q4K>(input, weights, output, rows, output_features, input_features, false, stream);
}

MOTE_EXPORT int mote_hip_quantized_linear_q4_k_f16(const void* input, const void* weights, void* output,
                                                  uint64_t rows, uint64_t output_features,
                                                  uint64_t input_features, void* stream) noexcept {
    return mote::kquant::linear<Fmt::Q4K>(input, weights, output, rows, output_features, input_features, true, stream);
}

MOTE_EXPORT int mote_hip_quantized_linear_q6_k_f32(const void* input, const void* weights, void* output,
                                                  uint64_t rows, uint64_t output_features,
                                                  uint64_t input_features, void* stream) noexcept {
    return mote::kquant::linear<Fmt::Q6K>(input, weights, output, rows, output_features, input_features, false, stream);
}

MOTE_EXPORT int mote_hip_quantized_linear_q6_k_f16(const void* input, const void* weights, void* output,
                                                  uint64_t rows, uint64_t output_features,
                                                  uint64_t input_features, void* stream) noexcept {
    return mote::kquant::linear<Fmt::Q6K>(input, weights, output, rows, output_features, input_features, true, stream);
}

MOTE_EXPORT int mote_hip_dequantize_q4_k_f32(const void* weights, void* output, uint64_t rows,
                                            uint64_t input_features, void* stream) noexcept {
    return mote::kquant::dequantize<Fmt::Q4K>(weights, output, rows, input_features, stream);
}

MOTE_EXPORT int mote_hip_dequantize_q6_k_f32(const void* weights, void* output, uint64_t rows,
                                            uint64_t input_features, void* stream) noexcept {
    return mote::kquant::dequantize<Fmt::Q6K>(weights, output, rows, input_features, stream);
}

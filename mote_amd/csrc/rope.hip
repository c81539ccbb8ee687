// Rotary position embedding, f16 in/out with f32 cos/sin tables.
//
// For each (token, head) vector and pair j < rotary_dim / 2 with the
// half-split pairing (first = j, second = j + R/2) or the interleaved pairing
// (first = 2j, second = 2j + 1):
//   out[first]  = f16(a * cos[t, j] - b * sin[t, j])
//   out[second] = f16(b * cos[t, j] + a * sin[t, j])
// and elements [rotary_dim, head_dim) are copied bit for bit.  Kernel and shim
// semantics: crates/mote-backend-hip/src/rope.hip:35-150; oracle
// crates/mote-reference/src/lib.rs:170-244.
//
// A thread owns four rotation pairs (two 8-byte loads for the half-split
// layout, one 16-byte load for interleaved, 16-byte cos/sin loads) or four
// tail elements; each element is read and written by the same thread, so
// input == output is race free.  Shapes or pointers that do not allow the
// vector form fall back to one thread per pair / tail element.  The fused
// entry point rotates q and k, which share the token's cos/sin row, in one
// launch.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"

namespace mote::rope {
namespace {

constexpr int kInvalid = -1;
constexpr uint64_t kMaxGridX = 0xffffffffull;
constexpr uint32_t kHalfSplit = 0;
constexpr uint32_t kInterleaved = 1;

struct Geometry {
    uint64_t tokens, heads_a, heads_b, head_dim, rotary_dim;
    uint32_t layout;
};

// Returns (f16(a c - b s), f16(b c + a s)).
__device__ __forceinline__ f16x2 rotate(float a, float b, float c, float s) {
    return f16x2{static_cast<_Float16>(a * c - b * s), static_cast<_Float16>(b * c + a * s)};
}

// Vector path: items per vector = R/8 rotation quads + tail/4 copy quads.
// Idx is the index type: 32-bit when every item index fits (the divisions
// that locate an item's vector and token are then hardware 32-bit ones, not
// the multi-instruction 64-bit sequence in front of every load).
template <uint32_t LAYOUT, typename Idx>
__global__ __launch_bounds__(256) void rope_vec_kernel(const _Float16* in_a, const _Float16* in_b,
                                                       const float* __restrict__ cos_t,
                                                       const float* __restrict__ sin_t,
                                                       _Float16* out_a, _Float16* out_b,
                                                       uint64_t vectors_a, uint64_t total_items,
                                                       uint32_t heads_a, uint32_t heads_b,
                                                       uint32_t head_dim, uint32_t rotary_dim) {
    const uint32_t freq = rotary_dim / 2;
    const uint32_t rot_items = freq / 4;
    const uint32_t items = rot_items + (head_dim - rotary_dim) / 4;
    const Idx stride = static_cast<Idx>(gridDim.x) * 256;
    for (Idx it = static_cast<Idx>(blockIdx.x) * 256 + threadIdx.x; it < static_cast<Idx>(total_items);
         it += stride) {
        const Idx vec = it / items;
        const uint32_t item = static_cast<uint32_t>(it - vec * items);
        const bool is_a = vec < static_cast<Idx>(vectors_a);
        const Idx local = is_a ? vec : vec - static_cast<Idx>(vectors_a);
        const uint64_t token = local / (is_a ? heads_a : heads_b);
        const _Float16* src = (is_a ? in_a : in_b) + static_cast<uint64_t>(local) * head_dim;
        _Float16* dst = (is_a ? out_a : out_b) + static_cast<uint64_t>(local) * head_dim;
        if (item >= rot_items) {
            const uint32_t e = rotary_dim + (item - rot_items) * 4;
            *reinterpret_cast<u32x2*>(dst + e) = *reinterpret_cast<const u32x2*>(src + e);
            continue;
        }
        const uint32_t j = item * 4;
        const f32x4 c = *reinterpret_cast<const f32x4*>(cos_t + token * freq + j);
        const f32x4 s = *reinterpret_cast<const f32x4*>(sin_t + token * freq + j);
        if constexpr (LAYOUT == kHalfSplit) {
            const u32x2 av = *reinterpret_cast<const u32x2*>(src + j);
            const u32x2 bv = *reinterpret_cast<const u32x2*>(src + j + freq);
            const f16x2 a0 = as_h2(av.x), a1 = as_h2(av.y), b0 = as_h2(bv.x), b1 = as_h2(bv.y);
            const float a[4] = {static_cast<float>(a0.x), static_cast<float>(a0.y),
                                static_cast<float>(a1.x), static_cast<float>(a1.y)};
            const float b[4] = {static_cast<float>(b0.x), static_cast<float>(b0.y),
                                static_cast<float>(b1.x), static_cast<float>(b1.y)};
            const f16x2 r0 = rotate(a[0], b[0], c.x, s.x), r1 = rotate(a[1], b[1], c.y, s.y);
            const f16x2 r2 = rotate(a[2], b[2], c.z, s.z), r3 = rotate(a[3], b[3], c.w, s.w);
            const f16x2 oa[2] = {f16x2{r0.x, r1.x}, f16x2{r2.x, r3.x}};
            const f16x2 ob[2] = {f16x2{r0.y, r1.y}, f16x2{r2.y, r3.y}};
            *reinterpret_cast<u32x2*>(dst + j) =
                u32x2{__builtin_bit_cast(uint32_t, oa[0]), __builtin_bit_cast(uint32_t, oa[1])};
            *reinterpret_cast<u32x2*>(dst + j + freq) =
                u32x2{__builtin_bit_cast(uint32_t, ob[0]), __builtin_bit_cast(uint32_t, ob[1])};
        } else {
            const u32x4 v = *reinterpret_cast<const u32x4*>(src + 2 * j);
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
            const float cc[4] = {c.x, c.y, c.z, c.w};
            const float ss[4] = {s.x, s.y, s.z, s.w};
            uint32_t o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const f16x2 h = as_h2(w[i]);
                const f16x2 r = rotate(static_cast<float>(h.x), static_cast<float>(h.y), cc[i], ss[i]);
                o[i] = __builtin_bit_cast(uint32_t, r);
            }
            *reinterpret_cast<u32x4*>(dst + 2 * j) = u32x4{o[0], o[1], o[2], o[3]};
        }
    }
}

// Scalar path: items per vector = R/2 pairs + tail elements.
__global__ __launch_bounds__(256) void rope_scalar_kernel(const _Float16* in_a, const _Float16* in_b,
                                                          const float* __restrict__ cos_t,
                                                          const float* __restrict__ sin_t,
                                                          _Float16* out_a, _Float16* out_b,
                                                          uint64_t vectors_a, uint64_t total_items,
                                                          uint64_t heads_a, uint64_t heads_b,
                                                          uint64_t head_dim, uint64_t rotary_dim,
                                                          uint32_t layout) {
    const uint64_t freq = rotary_dim / 2;
    const uint64_t items = freq + (head_dim - rotary_dim);
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * 256;
    for (uint64_t it = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x; it < total_items;
         it += stride) {
        const uint64_t vec = it / items;
        const uint64_t item = it - vec * items;
        const bool is_a = vec < vectors_a;
        const uint64_t local = is_a ? vec : vec - vectors_a;
        const uint64_t token = local / (is_a ? heads_a : heads_b);
        const _Float16* src = (is_a ? in_a : in_b) + local * head_dim;
        _Float16* dst = (is_a ? out_a : out_b) + local * head_dim;
        if (item >= freq) {
            const uint64_t e = rotary_dim + (item - freq);
            dst[e] = src[e];
            continue;
        }
        const uint64_t first = layout == kHalfSplit ? item : 2 * item;
        const uint64_t second = layout == kHalfSplit ? item + freq : 2 * item + 1;
        const float a = static_cast<float>(src[first]);
        const float b = static_cast<float>(src[second]);
        const float c = cos_t[token * freq + item];
        const float s = sin_t[token * freq + item];
        const f16x2 r = rotate(a, b, c, s);
        dst[first] = r.x;
        dst[second] = r.y;
    }
}

bool aligned(const void* p, uintptr_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

int launch(const void* in_a, const void* in_b, const void* cos_t, const void* sin_t, void* out_a,
           void* out_b, const Geometry& g, hipStream_t stream) {
    const uint64_t vectors_a = g.tokens * g.heads_a;
    const uint64_t vectors = vectors_a + g.tokens * g.heads_b;
    const uint64_t freq = g.rotary_dim / 2;
    const uint64_t tail = g.head_dim - g.rotary_dim;
    const uintptr_t row_align = g.layout == kHalfSplit ? 8 : 16;
    bool vec = freq % 4 == 0 && tail % 4 == 0 && g.head_dim % (row_align / 2) == 0 &&
               g.head_dim <= 0xffffffffull && g.heads_a <= 0xffffffffull &&
               g.heads_b <= 0xffffffffull && (freq == 0 || (aligned(cos_t, 16) && aligned(sin_t, 16)));
    for (const void* p : {in_a, static_cast<const void*>(out_a)}) vec = vec && aligned(p, row_align);
    if (g.heads_b) {
        for (const void* p : {in_b, static_cast<const void*>(out_b)}) vec = vec && aligned(p, row_align);
    }
    const uint64_t items = vec ? freq / 4 + tail / 4 : freq + tail;
    const uint64_t total = vectors * items;
    if (total == 0) return 0;
    const uint64_t blocks64 = (total + 255) / 256;
    const dim3 grid(static_cast<unsigned>(blocks64 < 65536 ? blocks64 : 65536)), block(256);
    const auto* ia = static_cast<const _Float16*>(in_a);
    const auto* ib = static_cast<const _Float16*>(in_b);
    auto* oa = static_cast<_Float16*>(out_a);
    auto* ob = static_cast<_Float16*>(out_b);
    const auto* c = static_cast<const float*>(cos_t);
    const auto* s = static_cast<const float*>(sin_t);
    const uint64_t heads_b = g.heads_b == 0 ? 1 : g.heads_b;  // divisor of never-taken k path
    // 32-bit indices when the last item index plus one grid stride fits
    const bool narrow = total + static_cast<uint64_t>(grid.x) * 256 <= 0xffffffffull;
    auto launch_vec = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, block, 0, stream, ia, ib, c, s, oa, ob, vectors_a, total,
                           static_cast<uint32_t>(g.heads_a), static_cast<uint32_t>(heads_b),
                           static_cast<uint32_t>(g.head_dim), static_cast<uint32_t>(g.rotary_dim));
    };
    if (vec && g.layout == kHalfSplit) {
        if (narrow) launch_vec(rope_vec_kernel<kHalfSplit, uint32_t>);
        else launch_vec(rope_vec_kernel<kHalfSplit, uint64_t>);
    } else if (vec) {
        if (narrow) launch_vec(rope_vec_kernel<kInterleaved, uint32_t>);
        else launch_vec(rope_vec_kernel<kInterleaved, uint64_t>);
    } else {
        hipLaunchKernelGGL(rope_scalar_kernel, grid, block, 0, stream, ia, ib, c, s, oa, ob,
                           vectors_a, total, g.heads_a, heads_b, g.head_dim,
                           g.rotary_dim, g.layout);
    }
    return static_cast<int>(hipGetLastError());
}

__global__ __launch_bounds__(256) void tables_kernel(const int64_t* __restrict__ positions,
                                                     float* __restrict__ cos_t,
                                                     float* __restrict__ sin_t, uint64_t tokens,
                                                     uint64_t rotary_dim, double theta) {
    const uint64_t freq = rotary_dim / 2;
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= tokens * freq) return;
    const uint64_t t = i / freq, j = i - t * freq;
    const double inv = pow(theta, -(2.0 * static_cast<double>(j)) / static_cast<double>(rotary_dim));
    const double angle = static_cast<double>(positions[t]) * inv;
    cos_t[i] = static_cast<float>(cos(angle));
    sin_t[i] = static_cast<float>(sin(angle));
}

// Argument checks of crates/mote-backend-hip/src/rope.hip:109-130.
int check(const void* input, const void* cos_t, const void* sin_t, const void* output,
          uint64_t rotary_dim, uint64_t head_dim, uint32_t layout, const void* stream) {
    if (!input || !output || !stream) return kInvalid;
    if (rotary_dim > 0 && (!cos_t || !sin_t)) return kInvalid;
    if (layout != kHalfSplit && layout != kInterleaved) return kInvalid;
    if ((rotary_dim & 1u) != 0 || rotary_dim > head_dim) return kInvalid;
    return 1;
}

}  // namespace
}  // namespace mote::rope

MOTE_EXPORT int mote_hip_rope_f16(const void* input, const void* cos, const void* sin, void* output,
                                 uint64_t tokens, uint64_t heads, uint64_t head_dim,
                                 uint64_t rotary_dim, uint32_t layout, void* stream) noexcept {
    using namespace mote::rope;
    const int pre = check(input, cos, sin, output, rotary_dim, head_dim, layout, stream);
    if (pre != 1) return pre;
    if (tokens == 0 || heads == 0 || head_dim == 0) return 0;
    if (tokens > kMaxGridX / heads) return kInvalid;
    const Geometry g{tokens, heads, 0, head_dim, rotary_dim, layout};
    return launch(input, nullptr, cos, sin, output, nullptr, g, static_cast<hipStream_t>(stream));
}

// Fused q + k rotation: q [tokens, q_heads, head_dim] and k [tokens, k_heads,
// head_dim] share cos/sin [tokens, rotary_dim / 2].  No counterpart in the
// reference (it launches once per tensor).
MOTE_EXPORT int mote_hip_rope_qk_f16(const void* q_input, const void* k_input, const void* cos,
                                    const void* sin, void* q_output, void* k_output,
                                    uint64_t tokens, uint64_t q_heads, uint64_t k_heads,
                                    uint64_t head_dim, uint64_t rotary_dim, uint32_t layout,
                                    void* stream) noexcept {
    using namespace mote::rope;
    int pre = check(q_input, cos, sin, q_output, rotary_dim, head_dim, layout, stream);
    if (pre != 1) return pre;
    if (k_heads > 0 && (!k_input || !k_output)) return kInvalid;
    if (tokens == 0 || head_dim == 0 || (q_heads == 0 && k_heads == 0)) return 0;
    if (q_heads + k_heads < q_heads || tokens > kMaxGridX / (q_heads + k_heads)) return kInvalid;
    const Geometry g{tokens, q_heads, k_heads, head_dim, rotary_dim, layout};
    if (q_heads == 0) {
        const Geometry gk{tokens, k_heads, 0, head_dim, rotary_dim, layout};
        return launch(k_input, nullptr, cos, sin, k_output, nullptr, gk, static_cast<hipStream_t>(stream));
    }
    return launch(q_input, k_input, cos, sin, q_output, k_output, g, static_cast<hipStream_t>(stream));
}

// cos/sin tables [tokens, rotary_dim / 2] for theta-based RoPE, computed in
// binary64 and rounded to binary32: inv_j = theta^(-2j / rotary_dim),
// angle = position * inv_j.  No counterpart in the reference (its RoPE takes
// caller-built tables, crates/mote-reference/src/lib.rs:158-163).
MOTE_EXPORT int mote_hip_rope_tables_f32(const void* positions, void* cos_out, void* sin_out,
                                        uint64_t tokens, uint64_t rotary_dim, double theta,
                                        void* stream) noexcept {
    if (!positions || !cos_out || !sin_out || !stream) return mote::rope::kInvalid;
    if ((rotary_dim & 1u) != 0 || !(theta > 0.0)) return mote::rope::kInvalid;
    const uint64_t count = tokens * (rotary_dim / 2);
    if (count == 0) return 0;
    const uint64_t blocks = (count + 255) / 256;
    if (blocks > 0x7fffffffull) return mote::rope::kInvalid;
    hipLaunchKernelGGL(mote::rope::tables_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const int64_t*>(positions),
                       static_cast<float*>(cos_out), static_cast<float*>(sin_out), tokens, rotary_dim,
                       theta);
    return static_cast<int>(hipGetLastError());
}

// RMSNorm and fused residual-add + RMSNorm, f16 in/out with f32 arithmetic.
//
//   rms_norm:   y = f16(x * (1 / sqrt(mean(x^2) + eps)) * w)
//               crates/mote-backend-hip/src/rms_norm.hip:22-98,
//               oracle crates/mote-reference/src/lib.rs:262-301
//   fused:      s = x + r (f32); y = f16(s * (1 / sqrt(mean(s^2) + eps)) * w);
//               r <- f16(s)
//               crates/mote-backend-hip/src/fused_add_rms_norm.hip:34-138,
//               oracle crates/mote-reference/src/lib.rs:333-384
//
// One 256-thread workgroup per row.  When the row is a whole number of
// 16-byte chunks and every pointer is 16-byte aligned, each thread loads its
// chunks once into registers (dwordx4), the sum of squares is reduced by DPP
// inside each wave and through LDS across the four waves in a fixed order
// (deterministic), and the same registers produce the output: every read
// precedes the barrier and every write follows it, so input == output (and
// input == residual for the fused op) is race free.  A thread's loads (input,
// residual, weights) are all issued before any is waited for, unguarded
// (indices past the row re-read its last chunk and are not used): guarded by
// a branch each, the compiler waited for each load before issuing the next,
// and at 32 x 4096 RMSNorm took 2.26 us against 2.06 us.  Other rows (e.g.
// hidden 513) use a strided two-pass loop with the same reduction.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "common.hpp"

namespace mote::norm {
namespace {

constexpr int kInvalid = -1;
constexpr uint64_t kMaxGridX = 0xffffffffull;

__device__ __forceinline__ float block_sum(float v, float* lds) {
    v = wave_sum(v);
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    if ((threadIdx.x & 63) == 0) lds[wave] = v;
    __syncthreads();
    return (lds[0] + lds[1]) + (lds[2] + lds[3]);
}

__device__ __forceinline__ void unpack8(const u32x4& v, float (&f)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const f16x2 h = as_h2(w[i]);
        f[2 * i] = static_cast<float>(h.x);
        f[2 * i + 1] = static_cast<float>(h.y);
    }
}

__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const f16x2 h = {static_cast<_Float16>(f[2 * i]), static_cast<_Float16>(f[2 * i + 1])};
        w[i] = __builtin_bit_cast(uint32_t, h);
    }
    return u32x4{w[0], w[1], w[2], w[3]};
}

template <int CPT, bool FUSED>
__global__ __launch_bounds__(256) void norm_vec_kernel(const u32x4* input, u32x4* residual,
                                                       const u32x4* __restrict__ weight,
                                                       u32x4* output, uint32_t chunks,
                                                       float hidden, float epsilon) {
    __shared__ float lds[4];
    const size_t row = blockIdx.x;
    const u32x4* in = input + row * chunks;
    u32x4* res = FUSED ? residual + row * chunks : nullptr;
    u32x4* out = output + row * chunks;

    // Unconditional loads (indices past the row re-read its last chunk and
    // are not used), weights included, all in flight before the reduction.
    u32x4 wreg[CPT], xreg[CPT], rreg[CPT];
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const uint32_t idx = min(threadIdx.x + 256u * c, chunks - 1);
        xreg[c] = in[idx];
        if constexpr (FUSED) rreg[c] = res[idx];
        wreg[c] = weight[idx];
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the arithmetic
    float v[CPT][8];
    float partial = 0.0f;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const bool live = threadIdx.x + 256u * c < chunks;
        unpack8(xreg[c], v[c]);
        if constexpr (FUSED) {
            float r[8];
            unpack8(rreg[c], r);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[c][i] = v[c][i] + r[i];
        }
        float sq = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) sq = __builtin_fmaf(v[c][i], v[c][i], sq);
        partial += live ? sq : 0.0f;
    }
    const float sum = block_sum(partial, lds);
    const float inv_rms = 1.0f / sqrtf(sum / hidden + epsilon);
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        float wv[8], o[8];
        unpack8(wreg[c], wv);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (v[c][i] * inv_rms) * wv[i];
        xreg[c] = pack8(o);
        if constexpr (FUSED) rreg[c] = pack8(v[c]);
    }
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const uint32_t idx = threadIdx.x + 256u * c;
        if (idx < chunks) {
            out[idx] = xreg[c];
            if constexpr (FUSED) res[idx] = rreg[c];
        }
    }
}

template <bool FUSED>
__global__ __launch_bounds__(256) void norm_scalar_kernel(const _Float16* input, _Float16* residual,
                                                          const _Float16* __restrict__ weight,
                                                          _Float16* output, uint64_t hidden,
                                                          float epsilon) {
    __shared__ float lds[4];
    const size_t row = blockIdx.x;
    const _Float16* in = input + row * hidden;
    _Float16* res = FUSED ? residual + row * hidden : nullptr;
    _Float16* out = output + row * hidden;
    float partial = 0.0f;
    for (uint64_t i = threadIdx.x; i < hidden; i += 256) {
        float s = static_cast<float>(in[i]);
        if constexpr (FUSED) s = s + static_cast<float>(res[i]);
        partial = __builtin_fmaf(s, s, partial);
    }
    const float sum = block_sum(partial, lds);
    const float inv_rms = 1.0f / sqrtf(sum / static_cast<float>(hidden) + epsilon);
    for (uint64_t i = threadIdx.x; i < hidden; i += 256) {
        float s = static_cast<float>(in[i]);
        if constexpr (FUSED) s = s + static_cast<float>(res[i]);
        out[i] = static_cast<_Float16>((s * inv_rms) * static_cast<float>(weight[i]));
        if constexpr (FUSED) res[i] = static_cast<_Float16>(s);
    }
}

template <bool FUSED>
int launch(const void* input, void* residual, const void* weight, void* output, uint64_t rows,
           uint64_t hidden, float epsilon, hipStream_t stream) {
    const uint64_t chunks = hidden / 8;
    const bool aligned = hidden % 8 == 0 &&
                         (reinterpret_cast<uintptr_t>(input) | reinterpret_cast<uintptr_t>(weight) |
                          reinterpret_cast<uintptr_t>(output) |
                          reinterpret_cast<uintptr_t>(FUSED ? residual : output)) % 16 == 0;
    const dim3 grid(static_cast<unsigned>(rows)), block(256);
    const float hidden_f = static_cast<float>(hidden);
    auto vec = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, block, 0, stream, static_cast<const u32x4*>(input),
                           static_cast<u32x4*>(residual), static_cast<const u32x4*>(weight),
                           static_cast<u32x4*>(output), static_cast<uint32_t>(chunks), hidden_f,
                           epsilon);
    };
    if (aligned && chunks <= 256) {
        vec(norm_vec_kernel<1, FUSED>);
    } else if (aligned && chunks <= 512) {
        vec(norm_vec_kernel<2, FUSED>);
    } else if (aligned && chunks <= 1024) {
        vec(norm_vec_kernel<4, FUSED>);
    } else {
        hipLaunchKernelGGL(norm_scalar_kernel<FUSED>, grid, block, 0, stream,
                           static_cast<const _Float16*>(input), static_cast<_Float16*>(residual),
                           static_cast<const _Float16*>(weight), static_cast<_Float16*>(output),
                           hidden, epsilon);
    }
    return static_cast<int>(hipGetLastError());
}

}  // namespace
}  // namespace mote::norm

// crates/mote-backend-hip/src/rms_norm.hip:68-98: -1 for null pointers or a
// grid that does not fit grid.x; empty rows/hidden succeed without a launch.
MOTE_EXPORT int mote_hip_rms_norm_f16(const void* input, const void* weight, void* output,
                                     uint64_t rows, uint64_t hidden_size, float epsilon,
                                     void* stream) noexcept {
    if (!input || !weight || !output || !stream) return mote::norm::kInvalid;
    if (rows == 0 || hidden_size == 0) return 0;
    if (rows > mote::norm::kMaxGridX) return mote::norm::kInvalid;
    return mote::norm::launch<false>(input, nullptr, weight, output, rows, hidden_size, epsilon,
                                     static_cast<hipStream_t>(stream));
}

// crates/mote-backend-hip/src/fused_add_rms_norm.hip:99-138: additionally -1
// for a non-finite or negative epsilon and for output == residual.
MOTE_EXPORT int mote_hip_fused_add_rms_norm_f16(const void* input, void* residual,
                                               const void* weight, void* output, uint64_t rows,
                                               uint64_t hidden_size, float epsilon,
                                               void* stream) noexcept {
    if (!input || !residual || !weight || !output || !stream) return mote::norm::kInvalid;
    if (!std::isfinite(epsilon) || epsilon < 0.0f) return mote::norm::kInvalid;
    if (output == residual) return mote::norm::kInvalid;
    if (rows == 0 || hidden_size == 0) return 0;
    if (rows > mote::norm::kMaxGridX) return mote::norm::kInvalid;
    return mote::norm::launch<true>(input, residual, weight, output, rows, hidden_size, epsilon,
                                    static_cast<hipStream_t>(stream));
}

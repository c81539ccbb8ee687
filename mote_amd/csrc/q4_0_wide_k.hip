// Q4_0 / Q8_0 linear and the fused Q4_0 gate/up for K above 2^31 - 1, past
// the 32-bit K and element offsets of the tiled kernels.  The reference kernel
// takes 64-bit sizes and launches for any K % 32 == 0
// (crates/mote-backend-hip/src/quantized_linear.hip:13-52, 56-91); so does
// this path, with the per-element decode of the generic kernel
// (crates/mote-reference/src/quantized.rs:177-201: (q - 8) d, or q d for Q8_0)
// in f32 and 64-bit offsets throughout.
//
// A row of x is at least 4 GiB here, so each output's K blocks are cut into
// `parts` runs and spread over the chip: workgroup item (part, output) has its
// 256 threads stride over the run's blocks, sums its waves in a fixed order and
// writes one partial to the split-K scratch ([parts][M][N], a second copy for
// the up rows); a second kernel adds the parts in part order (deterministic)
// and writes the output (silu(g) u for the fused op).
#include "common.hpp"
#include "q4_0.hpp"

#include <algorithm>

namespace mote::q4_0 {
namespace {

constexpr uint32_t kWideThreads = 256;
constexpr uint32_t kWideWaves = kWideThreads / kWave;
constexpr uint64_t kWideMaxParts = 1024;
constexpr uint64_t kWideItems = 65536;  // (part, output) items a launch aims for
constexpr uint32_t kWideGroups = 8192;  // workgroups of the partial kernel at most

__device__ __forceinline__ float wide_half(const uint8_t* p) {
    return static_cast<float>(__builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t*>(p)));
}

__device__ __forceinline__ float wide_x(const uint16_t* p) {
    return static_cast<float>(__builtin_bit_cast(_Float16, *p));
}

// One 32-element block's products added to acc, in element order.
template <bool Q8>
__device__ __forceinline__ float wide_block(const uint16_t* xb, const uint8_t* blk, float acc) {
    const float d = wide_half(blk);
    if constexpr (Q8) {
        for (int j = 0; j < 32; ++j)
            acc = __builtin_fmaf(wide_x(xb + j), static_cast<float>(static_cast<int8_t>(blk[2 + j])) * d, acc);
    } else {
        for (int j = 0; j < 16; ++j) {
            const uint8_t q = blk[2 + j];
            acc = __builtin_fmaf(wide_x(xb + j), static_cast<float>(static_cast<int>(q & 15) - 8) * d, acc);
            acc = __builtin_fmaf(wide_x(xb + j + 16), static_cast<float>(static_cast<int>(q >> 4) - 8) * d, acc);
        }
    }
    return acc;
}

template <bool Q8, bool GU>
__global__ __launch_bounds__(kWideThreads) void wide_k_part_kernel(const uint16_t* __restrict__ x,
                                                                   const uint8_t* __restrict__ wg,
                                                                   const uint8_t* __restrict__ wu,
                                                                   float* __restrict__ part, uint32_t N,
                                                                   uint64_t K, uint32_t parts, uint64_t count) {
    constexpr uint64_t kBlockBytesOf = Q8 ? 34 : 18;
    __shared__ float sums[2][kWideWaves];
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid / kWave;
    const uint64_t blocks = K / 32;
    const uint64_t run = (blocks + parts - 1) / parts;
    const uint64_t row_bytes = blocks * kBlockBytesOf;
    const uint64_t items = count * parts;
    for (uint64_t item = blockIdx.x; item < items; item += gridDim.x) {  // uniform per workgroup
        const uint32_t pt = static_cast<uint32_t>(item % parts);
        const uint64_t o = item / parts;
        const uint64_t m = o / N, n = o % N;
        const uint16_t* xr = x + m * K;
        const uint8_t* rg = wg + n * row_bytes;
        const uint8_t* ru = GU ? wu + n * row_bytes : nullptr;
        const uint64_t b0 = static_cast<uint64_t>(pt) * run;
        const uint64_t b1 = b0 + run < blocks ? b0 + run : blocks;
        float g = 0.0f, u = 0.0f;
        for (uint64_t b = b0 + tid; b < b1; b += kWideThreads) {
            g = wide_block<Q8>(xr + 32 * b, rg + b * kBlockBytesOf, g);
            if constexpr (GU) u = wide_block<Q8>(xr + 32 * b, ru + b * kBlockBytesOf, u);
        }
        g = wave_sum(g);
        if constexpr (GU) u = wave_sum(u);
        if ((tid & (kWave - 1)) == 0) {
            sums[0][wave] = g;
            sums[1][wave] = u;
        }
        __syncthreads();
        if (tid == 0) {
            float s = sums[0][0];
            for (uint32_t w = 1; w < kWideWaves; ++w) s += sums[0][w];
            part[static_cast<uint64_t>(pt) * count + o] = s;
            if constexpr (GU) {
                float t = sums[1][0];
                for (uint32_t w = 1; w < kWideWaves; ++w) t += sums[1][w];
                part[(static_cast<uint64_t>(parts) + pt) * count + o] = t;
            }
        }
        __syncthreads();  // sums is rewritten by the next item
    }
}

template <typename OutT, bool GU>
__global__ __launch_bounds__(256) void wide_k_reduce_kernel(const float* __restrict__ part, uint32_t parts,
                                                            uint64_t count, OutT* __restrict__ y) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x; i < count;
         i += static_cast<uint64_t>(gridDim.x) * 256) {
        float s = part[i];
        for (uint32_t k = 1; k < parts; ++k) s += part[static_cast<uint64_t>(k) * count + i];
        if constexpr (GU) {
            const float* up = part + static_cast<uint64_t>(parts) * count;
            float t = up[i];
            for (uint32_t k = 1; k < parts; ++k) t += up[static_cast<uint64_t>(k) * count + i];
            s = silu(s) * t;
        }
        y[i] = to_out<OutT>(s);
    }
}

template <typename OutT, bool GU>
void launch_reduce(const float* part, uint32_t parts, uint64_t count, void* y, hipStream_t stream) {
    const uint64_t blocks = (count + 255) / 256;
    const dim3 grid(static_cast<uint32_t>(std::min<uint64_t>(blocks, 2048))), block(256);
    hipLaunchKernelGGL((wide_k_reduce_kernel<OutT, GU>), grid, block, 0, stream, part, parts, count,
                       static_cast<OutT*>(y));
}

}  // namespace

hipError_t launch_wide_k(const Problem& p, uint64_t k, bool q8) {
    const bool gu = p.w_up != nullptr;
    if (gu && q8) return hipErrorInvalidValue;  // the fused op is Q4_0 only
    const uint64_t count = static_cast<uint64_t>(p.M) * p.N;
    if (count == 0) return hipSuccess;
    const uint32_t parts = static_cast<uint32_t>(
        std::clamp<uint64_t>((kWideItems + count - 1) / count, 1, std::min<uint64_t>(kWideMaxParts, k / 32)));
    const size_t need = kSplitKCounterBytes + count * parts * (gu ? 2 : 1) * sizeof(float);
    // The partials go after the split-K counter area of the scratch, which a
    // fresh pool buffer gets cleared, as for the split-K tiles.
    ScratchPool::Lease lease;
    uint8_t* base = nullptr;
    if (p.scratch != nullptr) {
        if (need > p.scratch_bytes) return hipErrorOutOfMemory;
        base = reinterpret_cast<uint8_t*>(p.scratch);
    } else {
        const hipError_t e = acquire_scratch(p.stream, need, &lease);
        if (e != hipSuccess) return e;
        base = static_cast<uint8_t*>(lease.ptr());
        if (lease.fresh()) {
            const hipError_t z = launch_zero_fill(base, kSplitKCounterBytes / 4, OutType::F32, p.stream);
            if (z != hipSuccess) return z;
        }
    }
    float* part = reinterpret_cast<float*>(base + kSplitKCounterBytes);
    const uint64_t items = count * parts;
    const dim3 grid(static_cast<uint32_t>(std::min<uint64_t>(items, kWideGroups))), block(kWideThreads);
    const auto* x = static_cast<const uint16_t*>(p.x);
    const auto* wg = static_cast<const uint8_t*>(p.w);
    const auto* wu = static_cast<const uint8_t*>(p.w_up);
    if (q8)
        hipLaunchKernelGGL((wide_k_part_kernel<true, false>), grid, block, 0, p.stream, x, wg, wu, part, p.N, k,
                           parts, count);
    else if (gu)
        hipLaunchKernelGGL((wide_k_part_kernel<false, true>), grid, block, 0, p.stream, x, wg, wu, part, p.N, k,
                           parts, count);
    else
        hipLaunchKernelGGL((wide_k_part_kernel<false, false>), grid, block, 0, p.stream, x, wg, wu, part, p.N, k,
                           parts, count);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (p.out == OutType::F32) {
        if (gu) launch_reduce<float, true>(part, parts, count, p.y, p.stream);
        else launch_reduce<float, false>(part, parts, count, p.y, p.stream);
    } else {
        if (gu) launch_reduce<_Float16, true>(part, parts, count, p.y, p.stream);
        else launch_reduce<_Float16, false>(part, parts, count, p.y, p.stream);
    }
    return hipGetLastError();
}

}  // namespace mote::q4_0

// Q4_0 support kernels: the alignment-agnostic fallback linear, the on-device
// block decoder and the K == 0 zero fill.
//
//  * q8_generic_kernel: the same for Q8_0 weights (34-byte blocks).
//  * generic_kernel: any K % 32 == 0 and any 2-byte-aligned pointers (the
//    Q4_0 storage alignment of crates/mote-types/src/lib.rs:67-73).  One wave
//    per weight row, lanes over 32-element blocks, the decode of
//    crates/mote-reference/src/quantized.rs:177-201 done per element in f32.
//    Used when the vectorised kernels' alignment or K % 64 conditions fail.
//  * decode kernels: write the f32 decode of every element.  The pair kernel
//    runs the same nibble unpack as the GEMV (1 + n/64 in binary16, then
//    (v - 1.125) * 64 = n - 8 exactly) so the element order and arithmetic of
//    the hot path are checked bit for bit against the oracle's
//    dequantize_quantized_row (crates/mote-reference/src/quantized.rs:58-74).
//  * zero fill: the reference launches its kernel for K == 0 and writes zeros
//    (crates/mote-backend-hip/tests/quantized_linear.rs:142-158); a fill
//    kernel is used rather than a memset so the call stays graph-capturable.
#include "common.hpp"
#include "q4_0.hpp"

namespace mote::q4_0 {
namespace {

__device__ __forceinline__ float load_half(const uint8_t* p) {
    const uint16_t bits = *reinterpret_cast<const uint16_t*>(p);
    return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

template <bool GATE_UP, typename OutT>
__global__ __launch_bounds__(256) void generic_kernel(const uint16_t* __restrict__ x,
                                                      const uint8_t* __restrict__ wg,
                                                      const uint8_t* __restrict__ wu,
                                                      OutT* __restrict__ y, uint32_t M,
                                                      uint32_t N, uint32_t K) {
    const uint32_t n = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = static_cast<int>(threadIdx.x) & 63;
    if (n >= N) return;
    const uint32_t blocks = K / kBlockElements;
    const size_t row_bytes = static_cast<size_t>(blocks) * kBlockBytes;
    const uint8_t* rg = wg + static_cast<size_t>(n) * row_bytes;
    const uint8_t* ru = GATE_UP ? wu + static_cast<size_t>(n) * row_bytes : nullptr;
    for (uint32_t m = blockIdx.y; m < M; m += gridDim.y) {
        const uint16_t* xr = x + static_cast<size_t>(m) * K;
        float g = 0.0f, u = 0.0f;
        for (uint32_t b = lane; b < blocks; b += kWave) {
            const uint8_t* bg = rg + static_cast<size_t>(b) * kBlockBytes;
            const float dg = load_half(bg);
            const uint8_t* bu = GATE_UP ? ru + static_cast<size_t>(b) * kBlockBytes : nullptr;
            const float du = GATE_UP ? load_half(bu) : 0.0f;
            for (int j = 0; j < 16; ++j) {
                const float x_lo = static_cast<float>(__builtin_bit_cast(_Float16, xr[32 * b + j]));
                const float x_hi = static_cast<float>(__builtin_bit_cast(_Float16, xr[32 * b + j + 16]));
                const uint8_t qg = bg[2 + j];
                g = __builtin_fmaf(x_lo, static_cast<float>(static_cast<int>(qg & 15) - 8) * dg, g);
                g = __builtin_fmaf(x_hi, static_cast<float>(static_cast<int>(qg >> 4) - 8) * dg, g);
                if constexpr (GATE_UP) {
                    const uint8_t qu = bu[2 + j];
                    u = __builtin_fmaf(x_lo, static_cast<float>(static_cast<int>(qu & 15) - 8) * du, u);
                    u = __builtin_fmaf(x_hi, static_cast<float>(static_cast<int>(qu >> 4) - 8) * du, u);
                }
            }
        }
        g = wave_sum(g);
        float v = g;
        if constexpr (GATE_UP) {
            u = wave_sum(u);
            v = silu(g) * u;
        }
        if (lane == 0) y[static_cast<size_t>(m) * N + n] = to_out<OutT>(v);
    }
}

template <bool GATE_UP>
hipError_t launch_generic(const Problem& p) {
    const dim3 grid((p.N + 3) / 4, min(p.M, 1024u)), block(256);
    if (p.out == OutType::F32) {
        hipLaunchKernelGGL((generic_kernel<GATE_UP, float>), grid, block, 0, p.stream,
                           static_cast<const uint16_t*>(p.x), static_cast<const uint8_t*>(p.w),
                           static_cast<const uint8_t*>(p.w_up), static_cast<float*>(p.y), p.M,
                           p.N, p.K);
    } else {
        hipLaunchKernelGGL((generic_kernel<GATE_UP, _Float16>), grid, block, 0, p.stream,
                           static_cast<const uint16_t*>(p.x), static_cast<const uint8_t*>(p.w),
                           static_cast<const uint8_t*>(p.w_up), static_cast<_Float16*>(p.y), p.M,
                           p.N, p.K);
    }
    return hipGetLastError();
}

// Q8_0 (crates/mote-reference/src/quantized.rs:191-195): 34-byte blocks, an f16
// scale and 32 two's-complement bytes, value v d.  Same mapping as the Q4_0
// generic kernel: one wave per weight row, lanes over blocks, f32 arithmetic.
template <typename OutT>
__global__ __launch_bounds__(256) void q8_generic_kernel(const uint16_t* __restrict__ x,
                                                         const uint8_t* __restrict__ w,
                                                         OutT* __restrict__ y, uint32_t M,
                                                         uint32_t N, uint32_t K) {
    constexpr uint32_t kQ8BlockBytes = 34;
    const uint32_t n = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = static_cast<int>(threadIdx.x) & 63;
    if (n >= N) return;
    const uint32_t blocks = K / kBlockElements;
    const uint8_t* row = w + static_cast<size_t>(n) * blocks * kQ8BlockBytes;
    for (uint32_t m = blockIdx.y; m < M; m += gridDim.y) {
        const uint16_t* xr = x + static_cast<size_t>(m) * K;
        float acc = 0.0f;
        for (uint32_t b = lane; b < blocks; b += kWave) {
            const uint8_t* blk = row + static_cast<size_t>(b) * kQ8BlockBytes;
            const float d = load_half(blk);
            for (int j = 0; j < 32; ++j) {
                const float xv = static_cast<float>(__builtin_bit_cast(_Float16, xr[32 * b + j]));
                acc = __builtin_fmaf(xv, static_cast<float>(static_cast<int8_t>(blk[2 + j])) * d, acc);
            }
        }
        acc = wave_sum(acc);
        if (lane == 0) y[static_cast<size_t>(m) * N + n] = to_out<OutT>(acc);
    }
}

hipError_t launch_q8_generic(const Problem& p) {
    const dim3 grid((p.N + 3) / 4, min(p.M, 1024u)), block(256);
    if (p.out == OutType::F32) {
        hipLaunchKernelGGL((q8_generic_kernel<float>), grid, block, 0, p.stream,
                           static_cast<const uint16_t*>(p.x), static_cast<const uint8_t*>(p.w),
                           static_cast<float*>(p.y), p.M, p.N, p.K);
    } else {
        hipLaunchKernelGGL((q8_generic_kernel<_Float16>), grid, block, 0, p.stream,
                           static_cast<const uint16_t*>(p.x), static_cast<const uint8_t*>(p.w),
                           static_cast<_Float16*>(p.y), p.M, p.N, p.K);
    }
    return hipGetLastError();
}

const Variant kGeneric[] = {
    Variant{"generic", Kind::Generic, 0, 0, 0, &launch_generic<false>},
    Variant{"gateup_generic", Kind::GateUpGeneric, 0, 0, 0, &launch_generic<true>},
    Variant{"q8_generic", Kind::Q8Generic, 0, 0, 0, &launch_q8_generic},
};

// One thread per block pair; same unpack as the GEMV kernel.
__global__ __launch_bounds__(256) void decode_pairs_kernel(const uint8_t* __restrict__ w,
                                                           float* __restrict__ out,
                                                           uint64_t pairs) {
    const uint64_t p = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (p >= pairs) return;
    uint32_t d[9];
    load_pair(w + p * kPairBytes, d);
    uint32_t q[8];
    q[0] = pair_q0(d);
    q[1] = d[1]; q[2] = d[2]; q[3] = d[3];
    q[4] = d[5]; q[5] = d[6]; q[6] = d[7]; q[7] = d[8];
    const float scale[2] = {half_lo_to_float(d[0]), half_hi_to_float(d[4])};
    float* o = out + p * 64;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int base = i < 4 ? 0 : 32;
        const float s = scale[i < 4 ? 0 : 1];
        const uint32_t u[4] = {nib_hi02(q[i]), nib_lo02(q[i]), nib_lo13(q[i]), nib_hi13(q[i])};
        // element of the low / high half of each packed pair
        const int e0 = pair_byte_element(i, 0), e1 = pair_byte_element(i, 1);
        const int e2 = pair_byte_element(i, 2), e3 = pair_byte_element(i, 3);
        const int lo[4] = {e0 + 16, e0, e1, e1 + 16};
        const int hi[4] = {e2 + 16, e2, e3, e3 + 16};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const f16x2 h = as_h2(u[j]);
            const float vlo = (static_cast<float>(h.x) - 1.125f) * 64.0f;
            const float vhi = (static_cast<float>(h.y) - 1.125f) * 64.0f;
            o[base + lo[j]] = vlo * s;
            o[base + hi[j]] = vhi * s;
        }
    }
}

// One thread per block, byte loads: any K % 32 == 0, 2-byte-aligned storage.
__global__ __launch_bounds__(256) void decode_blocks_kernel(const uint8_t* __restrict__ w,
                                                            float* __restrict__ out,
                                                            uint64_t blocks) {
    const uint64_t b = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (b >= blocks) return;
    const uint8_t* blk = w + b * kBlockBytes;
    const float s = load_half(blk);
    float* o = out + b * kBlockElements;
    for (int j = 0; j < 16; ++j) {
        const uint8_t q = blk[2 + j];
        o[j] = static_cast<float>(static_cast<int>(q & 15) - 8) * s;
        o[j + 16] = static_cast<float>(static_cast<int>(q >> 4) - 8) * s;
    }
}

template <typename T>
__global__ __launch_bounds__(256) void zero_kernel(T* __restrict__ y, uint64_t count) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * 256;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x; i < count; i += stride)
        y[i] = T(0);
}

}  // namespace

const Variant* generic_variants(int* count) {
    *count = static_cast<int>(sizeof(kGeneric) / sizeof(kGeneric[0]));
    return kGeneric;
}

hipError_t launch_zero_fill(void* y, uint64_t count, OutType out, hipStream_t stream) {
    if (count == 0) return hipSuccess;
    const uint64_t blocks = (count + 255) / 256;
    const dim3 grid(static_cast<unsigned>(blocks < 65536 ? blocks : 65536)), block(256);
    if (out == OutType::F32) {
        hipLaunchKernelGGL(zero_kernel<float>, grid, block, 0, stream, static_cast<float*>(y), count);
    } else {
        hipLaunchKernelGGL(zero_kernel<_Float16>, grid, block, 0, stream, static_cast<_Float16*>(y), count);
    }
    return hipGetLastError();
}

hipError_t launch_decode_f32(const void* w, float* out, uint64_t rows, uint64_t cols,
                             hipStream_t stream) {
    const uint64_t blocks = rows * (cols / kBlockElements);
    if (blocks == 0) return hipSuccess;
    const bool pairs_ok = cols % 64 == 0 && reinterpret_cast<uintptr_t>(w) % 4 == 0;
    if (pairs_ok) {
        const uint64_t pairs = blocks / 2;
        const uint64_t grid = (pairs + 255) / 256;
        if (grid > 0x7fffffffull) return hipErrorInvalidConfiguration;
        hipLaunchKernelGGL(decode_pairs_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                           stream, static_cast<const uint8_t*>(w), out, pairs);
    } else {
        const uint64_t grid = (blocks + 255) / 256;
        if (grid > 0x7fffffffull) return hipErrorInvalidConfiguration;
        hipLaunchKernelGGL(decode_blocks_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                           stream, static_cast<const uint8_t*>(w), out, blocks);
    }
    return hipGetLastError();
}

}  // namespace mote::q4_0

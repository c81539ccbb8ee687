// HBM read probe: a pure-read kernel that measures the read floor the
// quantized GEMVs are held against (bench.py --read-floor).  It is built into
// its own library, libmote_probe.so, which only the benchmark loads: it is a
// measuring instrument, not part of the drop-in C ABI of libmote_hip.so.
//
// Grid-stride 16-byte loads: thread t of a grid of T threads reads chunks
// t, t + T, t + 2T, ... of the buffer, `in_flight` loads per thread issued
// before any is used, optionally non-temporal.  The values are folded into
// one word that is stored only if it equals a constant no buffer here
// produces, so the loads stay live and nothing is written in practice.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"
#include "export.hpp"

namespace mote {
namespace {

template <int THREADS, int UNROLL, bool NT>
__global__ __launch_bounds__(THREADS) void read_probe_kernel(const u32x4* __restrict__ p, uint64_t n16,
                                                             uint32_t* __restrict__ sink) {
    uint32_t acc = 0;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * THREADS;
    uint64_t i = static_cast<uint64_t>(blockIdx.x) * THREADS + threadIdx.x;
    for (; i + (UNROLL - 1) * stride < n16; i += UNROLL * stride) {
        u32x4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) v[u] = NT ? __builtin_nontemporal_load(p + i + u * stride) : p[i + u * stride];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) acc = acc * 3u + (v[u].x ^ v[u].y ^ v[u].z ^ v[u].w);
    }
    for (; i < n16; i += stride) {
        const u32x4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;
}

template <int THREADS, int UNROLL, bool NT>
hipError_t launch(const void* data, uint64_t n16, uint32_t grid, void* sink, hipStream_t stream) {
    hipLaunchKernelGGL((read_probe_kernel<THREADS, UNROLL, NT>), dim3(grid), dim3(THREADS), 0, stream,
                       static_cast<const u32x4*>(data), n16, static_cast<uint32_t*>(sink));
    return hipGetLastError();
}

template <int THREADS, bool NT>
hipError_t by_unroll(uint32_t in_flight, const void* data, uint64_t n16, uint32_t grid, void* sink,
                     hipStream_t stream) {
    switch (in_flight) {
        case 2: return launch<THREADS, 2, NT>(data, n16, grid, sink, stream);
        case 4: return launch<THREADS, 4, NT>(data, n16, grid, sink, stream);
        case 8: return launch<THREADS, 8, NT>(data, n16, grid, sink, stream);
        default: return hipErrorInvalidValue;
    }
}

template <bool NT>
hipError_t by_threads(uint32_t threads, uint32_t in_flight, const void* data, uint64_t n16, uint32_t grid,
                      void* sink, hipStream_t stream) {
    switch (threads) {
        case 256: return by_unroll<256, NT>(in_flight, data, n16, grid, sink, stream);
        case 512: return by_unroll<512, NT>(in_flight, data, n16, grid, sink, stream);
        case 1024: return by_unroll<1024, NT>(in_flight, data, n16, grid, sink, stream);
        default: return hipErrorInvalidValue;
    }
}

// The smallest kernel of the decoder-step neighbours' shape: one 256-thread
// workgroup per row copying its bytes (16 bytes per thread and round), no
// arithmetic.  Its graph-replayed duration is the floor under RMSNorm and
// RoPE at these sizes.
__global__ __launch_bounds__(256) void copy_rows_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                        uint32_t chunks_per_row) {
    const size_t base = static_cast<size_t>(blockIdx.x) * chunks_per_row;
    for (uint32_t c = threadIdx.x; c < chunks_per_row; c += 256) dst[base + c] = src[base + c];
}

}  // namespace
}  // namespace mote

// Reads `bytes` (a multiple of 16, data 16-byte aligned) with grid-stride
// 16-byte loads: `grid` workgroups of `threads` (256, 512 or 1024) threads,
// `in_flight` (2, 4 or 8) loads per thread before use, non-temporal when
// non_temporal != 0.  `sink` (4 bytes) is written only for one impossible
// fold value.  Status: hipError_t (1 for a bad argument).
MOTE_EXPORT int mote_probe_read_u128(const void* data, size_t bytes, uint32_t grid, uint32_t threads,
                                     uint32_t in_flight, int non_temporal, void* sink, void* stream) noexcept {
    if (data == nullptr || sink == nullptr || stream == nullptr || bytes % 16 != 0 || grid == 0 ||
        reinterpret_cast<uintptr_t>(data) % 16 != 0)
        return hipErrorInvalidValue;
    if (bytes == 0) return hipSuccess;
    const auto s = static_cast<hipStream_t>(stream);
    const uint64_t n16 = bytes / 16;
    return static_cast<int>(non_temporal ? mote::by_threads<true>(threads, in_flight, data, n16, grid, sink, s)
                                         : mote::by_threads<false>(threads, in_flight, data, n16, grid, sink, s));
}

// Copies rows x row_bytes bytes (row_bytes a multiple of 16, both pointers
// 16-byte aligned, no overlap) with one 256-thread workgroup per row.
// Status: hipError_t (1 for a bad argument).
MOTE_EXPORT int mote_probe_copy_rows(const void* src, void* dst, uint32_t rows, uint32_t row_bytes,
                                     void* stream) noexcept {
    if (src == nullptr || dst == nullptr || stream == nullptr || row_bytes % 16 != 0 ||
        reinterpret_cast<uintptr_t>(src) % 16 != 0 || reinterpret_cast<uintptr_t>(dst) % 16 != 0)
        return hipErrorInvalidValue;
    if (rows == 0 || row_bytes == 0) return hipSuccess;
    hipLaunchKernelGGL(mote::copy_rows_kernel, dim3(rows), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const mote::u32x4*>(src), static_cast<mote::u32x4*>(dst), row_bytes / 16);
    return static_cast<int>(hipGetLastError());
}

// Measuring probes of the decode GEMV through the per-wave LDS ring
// (q4_0_gemv_lds.hip), built into libmote_probe.so, which only the benchmark
// loads (bench.py --timeline, --read-floor).
//
//  * mote_probe_ring_timeline: the shipped kernel body (gemv_lds_body of
//    gemv_lds.hpp, Q4_0, one token, 2 ring slots, 1 row in flight, f32 out)
//    instantiated with a timeline policy: every wave records the 100 MHz
//    real-time clock at its start, once x is staged and its first rows are
//    issued, when each of its rows has landed in the ring, when each row's sum
//    is formed, and after its last store.  Row stamps are kept one per lane
//    (lane j % 64 holds row j's, one v_cndmask per stamp) and every stamp is
//    written by vector stores after the wave's last y store, so the loop runs
//    the shipped instruction stream plus one clock read per hook.
//  * mote_probe_ring_read: the ring's loads and nothing else -- the same grid,
//    row order, non-temporal 16-byte direct-to-LDS loads, 2 slots and 1 row in
//    flight, and the same waits, with no LDS reads, arithmetic or stores: the
//    read floor of this kernel's own access pattern.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"
#include "export.hpp"
#include "gemv_formats.hpp"
#include "gemv_lds.hpp"

namespace mote::probe {
namespace {

using q4_0::FmtQ4;
using q4_0::kThreads;
using q4_0::kWaves;

// The shipped headline kernel's ring: slots per wave and rows in flight.
constexpr uint32_t kSlots = 2, kDepth = 1;

// Words of one wave's record: begin, ready, end, rows, then 64 arrival and 64
// computed stamps (rows past 64 are not recorded).
constexpr uint32_t kRecordWords = 4 + 64 + 64;

struct WaveTimeline {
    uint32_t* base;
    uint32_t* rec = nullptr;
    uint32_t t_begin = 0, t_ready = 0, arr = 0, done = 0;

    __device__ static uint32_t now() { return static_cast<uint32_t>(__builtin_amdgcn_s_memrealtime()); }
    __device__ static uint32_t lane() { return threadIdx.x & 63u; }

    __device__ __forceinline__ void begin(uint32_t g) {
        t_begin = now();
        rec = base + static_cast<size_t>(g) * kRecordWords;
    }
    __device__ __forceinline__ void ready() { t_ready = now(); }
    __device__ __forceinline__ void arrived(uint32_t j) {
        const uint32_t t = now();
        arr = lane() == (j & 63u) ? t : arr;
    }
    __device__ __forceinline__ void computed(uint32_t j) {
        const uint32_t t = now();
        done = lane() == (j & 63u) ? t : done;
    }
    __device__ __forceinline__ void end(uint32_t nrows) {
        const uint32_t t = now();
        if (lane() == 0) {
            rec[0] = t_begin;
            rec[1] = t_ready;
            rec[2] = t;
            rec[3] = nrows;
        }
        if (lane() < min(nrows, 64u)) {
            rec[4 + lane()] = arr;
            rec[68 + lane()] = done;
        }
    }
};

template <int LOADS>
__global__ __launch_bounds__(kThreads) void ring_timeline_kernel(const uint16_t* __restrict__ x,
                                                                 const uint8_t* __restrict__ w, float* __restrict__ y,
                                                                 uint32_t N, uint32_t K, uint32_t total,
                                                                 uint32_t* __restrict__ stamps) {
    WaveTimeline tl{stamps};
    q4_0::gemv_lds_body<FmtQ4, 1, kSlots, kDepth, LOADS, float>(x, w, y, N, K, total, tl);
}

// The ring's loads alone (see the file comment), with the shipped headline
// kernel's slots and rows in flight.
template <int LOADS, bool STAMPS>
__global__ __launch_bounds__(kThreads) void ring_read_kernel(const uint8_t* __restrict__ w, uint32_t N, uint32_t K,
                                                             uint32_t total, uint32_t* __restrict__ stamps) {
    constexpr uint32_t R = kSlots, D = kDepth;
    extern __shared__ __attribute__((aligned(16))) uint8_t ring_lds[];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t row_bytes = (K >> 6) * FmtQ4::kPairBytes, chunks = row_bytes >> 4;
    uint8_t* ring = ring_lds + wave * R * row_bytes;
    const uint32_t g = blockIdx.x * kWaves + wave;
    const uint32_t nrows = g < N ? (N - 1 - g) / total + 1 : 0;
    const uint32_t last = g < N ? g + (nrows - 1) * total : N - 1;
    WaveTimeline tl{stamps};
    if constexpr (STAMPS) tl.begin(g);
    auto load_row = [&](uint32_t jj, uint32_t slot) {
        const uint8_t* src = w + static_cast<size_t>(min(g + jj * total, last)) * row_bytes;
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const uint32_t c = 64u * static_cast<uint32_t>(i) + lane;
            if (i + 1 < LOADS || c < chunks)
                __builtin_amdgcn_global_load_lds(src + 16u * c, (q4_0::lds_ptr)(ring + slot * row_bytes + 1024u * i), 16,
                                                 0, 2 /* non-temporal */);
        }
    };
    auto wait_rows = [&](uint32_t rows) {
        if (rows >= 2) __builtin_amdgcn_s_waitcnt(q4_0::vm_wait(LOADS * 2));
        else if (rows == 1) __builtin_amdgcn_s_waitcnt(q4_0::vm_wait(LOADS));
        else __builtin_amdgcn_s_waitcnt(q4_0::vm_wait(0));
    };
#pragma unroll
    for (uint32_t d = 0; d < D; ++d)
        if (d < nrows) load_row(d, d);
    for (uint32_t j = 0; j < nrows; ++j) {
        if (j + D < nrows) {
            load_row(j + D, (j + D) % R);
            __builtin_amdgcn_s_waitcnt(q4_0::vm_wait(LOADS * D));
        } else {
            wait_rows(nrows - 1 - j);
        }
        if constexpr (STAMPS) {
            tl.arrived(j);
            tl.computed(j);
        }
    }
    __builtin_amdgcn_s_waitcnt(q4_0::vm_wait(0));
    if constexpr (STAMPS) tl.end(nrows);
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

// The shipped launcher's grid: one workgroup of 8 waves per CU, none without
// a row.
uint32_t ring_groups(uint32_t n) {
    const uint32_t need = (n + kWaves - 1) / kWaves;
    const uint32_t cus = static_cast<uint32_t>(device_cus());
    return cus < need ? cus : need;
}

bool ring_args_ok(const void* w, uint32_t n, uint32_t k) {
    return w != nullptr && n > 0 && k > 0 && k % 256 == 0 && k <= 4096 && reinterpret_cast<uintptr_t>(w) % 16 == 0;
}

}  // namespace
}  // namespace mote::probe

// Words per wave record of mote_probe_ring_timeline.
MOTE_EXPORT uint32_t mote_probe_ring_record_words(void) noexcept { return mote::probe::kRecordWords; }

// Waves the ring kernel runs for N rows (the size of the stamp buffer is
// waves x record words x 4 bytes).
MOTE_EXPORT uint32_t mote_probe_ring_waves(uint32_t n) noexcept {
    return n == 0 ? 0 : mote::probe::ring_groups(n) * mote::q4_0::kWaves;
}

// y[n] = sum_k x[k] w[n, k] (Q4_0, one token, f32 out) through the shipped
// ring kernel body with per-wave timestamps into `stamps` (at least
// mote_probe_ring_waves(n) * mote_probe_ring_record_words() words).  K a
// multiple of 256 up to 4096, x and w 16-byte aligned.  Status: hipError_t.
MOTE_EXPORT int mote_probe_ring_timeline(const void* x, const void* w, void* y, uint32_t n, uint32_t k,
                                         void* stamps, size_t stamps_bytes, void* stream) noexcept {
    using namespace mote::probe;
    if (!ring_args_ok(w, n, k) || x == nullptr || y == nullptr || stamps == nullptr || stream == nullptr ||
        reinterpret_cast<uintptr_t>(x) % 16 != 0)
        return hipErrorInvalidValue;
    const uint32_t groups = ring_groups(n);
    if (stamps_bytes < static_cast<size_t>(groups) * mote::q4_0::kWaves * kRecordWords * 4) return hipErrorInvalidValue;
    const uint32_t row_bytes = k / 64 * mote::kPairBytes;
    const uint32_t loads = (row_bytes / 16 + 63) / 64;
    const size_t lds = static_cast<size_t>(mote::q4_0::kWaves) * kSlots * row_bytes;
    const uint32_t total = groups * mote::q4_0::kWaves;
    const auto s = static_cast<hipStream_t>(stream);
    const auto* xp = static_cast<const uint16_t*>(x);
    const auto* wp = static_cast<const uint8_t*>(w);
    auto* yp = static_cast<float*>(y);
    auto* st = static_cast<uint32_t*>(stamps);
    switch (loads) {
        case 1: hipLaunchKernelGGL(ring_timeline_kernel<1>, dim3(groups), dim3(kThreads), lds, s, xp, wp, yp, n, k, total, st); break;
        case 2: hipLaunchKernelGGL(ring_timeline_kernel<2>, dim3(groups), dim3(kThreads), lds, s, xp, wp, yp, n, k, total, st); break;
        default: hipLaunchKernelGGL(ring_timeline_kernel<3>, dim3(groups), dim3(kThreads), lds, s, xp, wp, yp, n, k, total, st); break;
    }
    return static_cast<int>(hipGetLastError());
}

// Reads the N x K Q4_0 matrix at `w` with the ring kernel's loads only (see
// the file comment).  K a multiple of 256 up to 4096, w 16-byte aligned.
// With `stamps` (null: none) every wave records its start, each row's landing
// (in both row slots of the record) and its end, as mote_probe_ring_timeline
// does.  Status: hipError_t.
MOTE_EXPORT int mote_probe_ring_read(const void* w, uint32_t n, uint32_t k, void* stamps, size_t stamps_bytes,
                                     void* stream) noexcept {
    using namespace mote::probe;
    if (!ring_args_ok(w, n, k) || stream == nullptr) return hipErrorInvalidValue;
    const uint32_t groups = ring_groups(n);
    if (stamps != nullptr && stamps_bytes < static_cast<size_t>(groups) * mote::q4_0::kWaves * kRecordWords * 4)
        return hipErrorInvalidValue;
    const uint32_t row_bytes = k / 64 * mote::kPairBytes;
    const uint32_t loads = (row_bytes / 16 + 63) / 64;
    const size_t lds = static_cast<size_t>(mote::q4_0::kWaves) * kSlots * row_bytes;
    const uint32_t total = groups * mote::q4_0::kWaves;
    const auto s = static_cast<hipStream_t>(stream);
    const auto* wp = static_cast<const uint8_t*>(w);
    auto* st = static_cast<uint32_t*>(stamps);
#define MOTE_RING_READ(L)                                                                                         \
    do {                                                                                                          \
        if (st)                                                                                                   \
            hipLaunchKernelGGL((ring_read_kernel<L, true>), dim3(groups), dim3(kThreads), lds, s, wp, n, k, total, st); \
        else                                                                                                      \
            hipLaunchKernelGGL((ring_read_kernel<L, false>), dim3(groups), dim3(kThreads), lds, s, wp, n, k, total, st); \
    } while (0)
    switch (loads) {
        case 1: MOTE_RING_READ(1); break;
        case 2: MOTE_RING_READ(2); break;
        default: MOTE_RING_READ(3); break;
    }
#undef MOTE_RING_READ
    return static_cast<int>(hipGetLastError());
}

// Timeline probe of the skinny matrix-core GEMM (q4_0_skinny_mfma.hip), built
// into libmote_probe.so, which only the benchmark loads (bench.py
// --timeline-skinny).
//
//  * mote_probe_skinny_timeline: the shipped kernel (skinny_mfma_kernel of
//    skinny_mfma.hpp in the form the library plans for 4-32 tokens at K =
//    4096: 16 waves of one K step each, transposed loads, up to four items per
//    workgroup reduced together, activations by whole lines and before the
//    weights, f32 out; variant skinny_mfma_k16_s1_t1_d1_g1_r1_tr_l4_c_w), on
//    the grid the library computes for it (skinny_grid), instantiated with a
//    timeline policy: every wave reads the 100 MHz real-time clock at its
//    start, once its activations are converted to MFMA operands, when each
//    item's weights have landed in its stage and when that item's MFMAs are
//    issued, after the workgroup's reduction and stores, and at its end.  The
//    stamps stay in registers and lane 0 writes them with vector stores at
//    the end, so the kernel runs the shipped instruction stream plus one clock
//    read per hook.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"
#include "export.hpp"
#include "skinny_mfma.hpp"

namespace mote::probe {
namespace {

constexpr int kKS = 16, kSteps = 1, kMT = 1, kRT = 1, kLazy = 4;
constexpr uint32_t kK = kKS * kSteps * 256;  // the K this form runs without split K

// One wave's record: begin, x ready, reduced, end, items, then the landed and
// issued stamps of up to kLazy items; 16 words.
constexpr uint32_t kRecordWords = 16;

struct SkinnyTimeline {
    uint32_t* base;
    uint32_t t_begin = 0, t_x = 0, t_red = 0, n_items = 0;
    uint32_t t_land[kLazy] = {}, t_issue[kLazy] = {};

    __device__ explicit SkinnyTimeline(uint32_t* stamps) : base(stamps) {}
    __device__ static uint32_t now() { return static_cast<uint32_t>(__builtin_amdgcn_s_memrealtime()); }

    __device__ __forceinline__ void begin() { t_begin = now(); }
    __device__ __forceinline__ void x_ready() { t_x = now(); }
    __device__ __forceinline__ void landed(int i) {
        t_land[i] = now();
        n_items = static_cast<uint32_t>(i + 1);
    }
    __device__ __forceinline__ void issued(int i) { t_issue[i] = now(); }
    __device__ __forceinline__ void reduced() { t_red = now(); }
    __device__ __forceinline__ void end() {
        const uint32_t t = now();
        if ((threadIdx.x & 63u) == 0) {
            const uint32_t wave = blockIdx.x * (blockDim.x / 64u) + threadIdx.x / 64u;
            uint32_t* rec = base + static_cast<size_t>(wave) * kRecordWords;
            rec[0] = t_begin;
            rec[1] = t_x;
            rec[2] = t_red;
            rec[3] = t;
            rec[4] = n_items;
#pragma unroll
            for (int i = 0; i < kLazy; ++i) {
                rec[5 + i] = t_land[i];
                rec[5 + kLazy + i] = t_issue[i];
            }
        }
    }
};

int cus() {
    static const int n = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
            v = 256;
        return v;
    }();
    return n;
}

q4_0::SkinnyGrid grid_of(uint32_t M, uint32_t N) {
    return q4_0::skinny_grid<kKS, kSteps, kMT, 1, kRT, kLazy, false, false>(M, N, kK, cus());
}

}  // namespace
}  // namespace mote::probe

using namespace mote::probe;

MOTE_EXPORT uint32_t mote_probe_skinny_record_words() { return kRecordWords; }

// Waves of the probe's grid for M x 4096 x N (0 when the shape does not fit).
MOTE_EXPORT uint32_t mote_probe_skinny_waves(uint32_t M, uint32_t N) {
    if (M == 0 || M > 64 || N == 0) return 0;
    const mote::q4_0::SkinnyGrid g = grid_of(M, N);
    return g.ok ? g.groups * kKS : 0;
}

// y[M, N] (f32) = x[M, 4096] (f16) times the Q4_0 weights w[N, 4096], with
// every wave's record written to `stamps` (at least waves x 16 words).
// Returns 1 for shapes the form does not run or a buffer too small, before
// any launch.
MOTE_EXPORT int mote_probe_skinny_timeline(const void* x, const void* w, void* y, uint32_t M, uint32_t N,
                                           uint32_t K, void* stamps, size_t stamps_bytes, void* stream) {
    if (x == nullptr || w == nullptr || y == nullptr || stamps == nullptr || K != kK || M == 0 || M > 64 ||
        N == 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(w) % 4 != 0)
        return 1;
    const mote::q4_0::SkinnyGrid g = grid_of(M, N);
    if (!g.ok || stamps_bytes < static_cast<size_t>(g.groups) * kKS * kRecordWords * 4) return 1;
    hipLaunchKernelGGL((mote::q4_0::skinny_mfma_kernel<kKS, kSteps, kMT, 1, kRT, true, float, kLazy, true, false,
                                                       false, true, false, SkinnyTimeline>),
                       dim3(g.groups), dim3(kKS * 64), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(x), static_cast<const uint8_t*>(w), nullptr,
                       static_cast<float*>(y), M, N, K, g.token_groups, g.items, g.per_xcd, nullptr, 1u,
                       static_cast<uint32_t*>(stamps));
    return static_cast<int>(hipGetLastError());
}

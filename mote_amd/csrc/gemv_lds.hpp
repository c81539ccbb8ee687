// The decode GEMV through a per-wave LDS ring (q4_0_gemv_lds.hip), as a
// device function templated on a timeline policy, so that the probe library
// can instantiate the very kernel the library ships with per-wave timestamps
// (mote_amd/probes/ring_probe.hip) while the shipped kernel instantiates the
// policy that does nothing (NoTimeline: every hook is empty, and the code is
// that of the kernel without hooks).
#pragma once

#include "common.hpp"
#include "gemv_formats.hpp"
#include "q4_0.hpp"

namespace mote::q4_0 {
namespace {

// Timeline hooks of gemv_lds_body: begin (wave start; g is the wave's row
// group), ready (x staged and the first rows issued), arrived / computed (row
// j landed in the ring / its sum formed), end (after the last store).
struct NoTimeline {
    __device__ __forceinline__ void begin(uint32_t) {}
    __device__ __forceinline__ void ready() {}
    __device__ __forceinline__ void arrived(uint32_t) {}
    __device__ __forceinline__ void computed(uint32_t) {}
    __device__ __forceinline__ void end(uint32_t) {}
};

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kWave;
constexpr uint32_t kMaxK = 4096;
typedef __attribute__((address_space(3))) void* lds_ptr;

// s_waitcnt immediate that waits until at most n vector memory loads are
// outstanding (vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt not waited).
constexpr int vm_wait(int n) { return (n & 0xF) | ((n >> 4) << 14) | 0x0F70; }


// F: the weight format (FmtQ4: 36-byte Q4_0 block pairs, FmtQ8: 68-byte Q8_0
// pairs); MT: tokens, every row read once for all of them (the pair's
// operands unpacked once and shared by the tokens' dot chains).  LOADS:
// 16-byte chunks of a row / 64, rounded up (Q4_0: 1 for K <= 1792, 2 up to
// 3584, 3 up to 4096; Q8_0: up to 5).
template <class F, int MT, int R, int D, int LOADS, typename OutT, class TL>
__device__ __forceinline__ void gemv_lds_body(const uint16_t* __restrict__ x, const uint8_t* __restrict__ w,
                                              OutT* __restrict__ y, uint32_t N, uint32_t K, uint32_t total_groups,
                                              TL& tl) {
    static_assert(D >= 1 && D <= 3 && D < R, "the ring holds the rows in flight and the one computed");
    static_assert(MT >= 1 && MT <= 4, "tokens per row read");
    extern __shared__ __attribute__((aligned(16))) uint8_t ring_lds[];  // [waves][R][row bytes]
    __shared__ __attribute__((aligned(16))) uint8_t xs[MT * kMaxK * 2];  // x of token m at 8 KB m
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const uint32_t npairs = K >> 6;
    const uint32_t row_bytes = npairs * F::kPairBytes;  // a multiple of 16: K % 256 == 0
    const uint32_t chunks = row_bytes >> 4;
    uint8_t* ring = ring_lds + static_cast<uint32_t>(wave) * R * row_bytes;
    const uint32_t g = blockIdx.x * kWaves + static_cast<uint32_t>(wave);
    const uint32_t nrows = g < N ? (N - 1 - g) / total_groups + 1 : 0;
    const uint32_t last = g < N ? g + (nrows - 1) * total_groups : N - 1;
    const uint32_t pc = min(static_cast<uint32_t>(lane), npairs - 1);
    const uint32_t keep = static_cast<uint32_t>(lane) < npairs ? 0xFFFFFFFFu : 0u;  // NaN-safe drop of idle lanes
    tl.begin(g);

    // Row jj (< nrows) of this wave into ring slot `slot`: chunk 64 i + lane
    // per instruction, the last instruction's lanes past the row idle.
    auto load_row = [&](uint32_t jj, uint32_t slot) {
        const uint8_t* src = w + static_cast<size_t>(min(g + jj * total_groups, last)) * row_bytes;
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const uint32_t c = 64u * static_cast<uint32_t>(i) + static_cast<uint32_t>(lane);
            if (i + 1 < LOADS || c < chunks)
                __builtin_amdgcn_global_load_lds(src + 16u * c, (lds_ptr)(ring + slot * row_bytes + 1024u * i), 16, 0,
                                                 2 /* non-temporal */);
        }
    };

    // x first: thread t loads 16-byte chunk t (clamped) of every token to xs
    // + 8 KB m + 16 t, and every wave's x loads are issued before any weight
    // load of the workgroup.
    // Swizzled: chunk 8 a + i of x (the i-th 16 bytes of pair a) sits at
    // position 8 a + ((i + a) & 7), so that the lanes reading their pairs'
    // 128 bytes below hit distinct banks (unswizzled, every lane of an
    // instruction reads the same bank row: 4096 x 4096 3.96 -> 3.66 us);
    // thread t fills position t.
    const uint32_t xc = min(swizzled_chunk(static_cast<uint32_t>(tid)), npairs * 8 - 1);
#pragma unroll
    for (int m = 0; m < MT; ++m)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t*>(x) + static_cast<size_t>(m) * K * 2 + 16u * xc,
                                         (lds_ptr)(xs + m * kMaxK * 2 + 1024u * static_cast<uint32_t>(wave)), 16, 0,
                                         0);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // Waits until at most `rows` rows' loads (rows <= D, wave-uniform) are
    // outstanding (vmcnt counts in issue order).
    auto wait_rows = [&](uint32_t rows) {
        if (rows >= 3 && D >= 3) __builtin_amdgcn_s_waitcnt(vm_wait(LOADS * 3));
        else if (rows == 2 && D >= 2) __builtin_amdgcn_s_waitcnt(vm_wait(LOADS * 2));
        else if (rows == 1) __builtin_amdgcn_s_waitcnt(vm_wait(LOADS));
        else __builtin_amdgcn_s_waitcnt(vm_wait(0));
    };
#pragma unroll
    for (int d = 0; d < D; ++d)
        if (static_cast<uint32_t>(d) < nrows) load_row(static_cast<uint32_t>(d), static_cast<uint32_t>(d));
    __builtin_amdgcn_sched_barrier(0);
    // no more than this wave's first rows' loads outstanding means its x
    // chunks have landed; the barrier then covers every wave's
    wait_rows(nrows < static_cast<uint32_t>(D) ? nrows : static_cast<uint32_t>(D));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    tl.ready();

    XPair xv[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        uint32_t xr[32];
        const uint8_t* slot = xs + m * kMaxK * 2 + pc * 128u;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(slot + ((static_cast<uint32_t>(i) + pc) & 7u) * 16u);
            xr[4 * i + 0] = v.x; xr[4 * i + 1] = v.y; xr[4 * i + 2] = v.z; xr[4 * i + 3] = v.w;
        }
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            s0 = dot2(xr[i], kOnePair, s0);
            s1 = dot2(xr[16 + i], kOnePair, s1);
        }
        xv[m].c0 = F::kStart * s0;
        xv[m].c1 = F::kStart * s1;
        F::order_x(xr, xv[m]);
    }

    // Row sums stay in lanes (lane j % 64 holds row j) and are stored every 64
    // rows and at the end.
    float mine[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) mine[m] = 0.0f;
    for (uint32_t j = 0; j < nrows; ++j) {
        // Rows are loaded only up to the wave's last, so the loads left in
        // flight once row j has landed shrink at the end.
        if (j + D < nrows) {
            load_row(j + D, (j + D) % R);
            __builtin_amdgcn_s_waitcnt(vm_wait(LOADS * D));
        } else {
            wait_rows(nrows - 1 - j);
        }
        tl.arrived(j);
        const uint32_t* pr = reinterpret_cast<const uint32_t*>(ring + (j % R) * row_bytes + pc * F::kPairBytes);
        uint32_t raw[F::kDwords];
#pragma unroll
        for (int i = 0; i < F::kDwords; ++i) raw[i] = pr[i];
        float part[MT];
        if constexpr (MT == 1) {
            part[0] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, F::dot(raw, xv[0])) & keep);
        } else {
            Unpacked wu;
            F::unpack(raw, wu);
#pragma unroll
            for (int m = 0; m < MT; ++m)
                part[m] = 0.0f + __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, F::dot(wu, xv[m])) & keep);
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float s = wave_sum(part[m]);
            if (__builtin_expect(not_finite(s), 0)) {  // wave-uniform: the reference's per-element sum
                const uint8_t* pair = w + static_cast<size_t>(g + j * total_groups) * row_bytes + pc * F::kPairBytes;
                const float e = keep != 0u ? F::exact(pair, x + static_cast<size_t>(m) * K + pc * 64u) : 0.0f;
                s = wave_sum(e) * (1.0f / F::kFinal);
            }
            mine[m] = static_cast<uint32_t>(lane) == (j & 63u) ? s : mine[m];
        }
        tl.computed(j);
        if ((j & 63u) == 63u || j + 1 == nrows) {
            const uint32_t first = j & ~63u;
            if (static_cast<uint32_t>(lane) <= (j & 63u)) {
                OutT* yr = y + g + (first + static_cast<uint32_t>(lane)) * total_groups;
#pragma unroll
                for (int m = 0; m < MT; ++m) yr[static_cast<size_t>(m) * N] = to_out<OutT>(F::kFinal * mine[m]);
            }
        }
    }
    tl.end(nrows);
}

}  // namespace
}  // namespace mote::q4_0

// Q4_0 decode GEMV (M = 1) for gfx950: persistent, software-pipelined waves.
//
// Computes y[n] = sum_k x[k] * w[n, k] for f16 x [K] and GGML Q4_0 w [N, K]
// (K <= 4096), the operation of crates/mote-backend-hip/src/
// quantized_linear.hip:13-52 (oracle crates/mote-reference/src/
// quantized.rs:89-144) at rows == 1.
//
// The grid is G workgroups of 8 waves per CU.  Lane l owns block pair l (64
// elements, 36 bytes) of every row; wave g of the grid walks rows g, g + W,
// g + 2W, ... (W waves in the grid), so at any moment the waves of the whole
// chip read neighbouring rows and the request front sweeps the matrix once,
// in order.  Each wave keeps D rows in flight: it computes row j while the
// loads of rows j + 1 .. j + D - 1 are outstanding and issues row j + D right
// after, so the nibble arithmetic of early rows overlaps the HBM stream of
// later ones instead of piling up after the last byte arrives.
//
// x is staged once per workgroup through LDS (coalesced 16-byte loads, one
// 144-byte slot per 128-byte pair chunk so the per-lane reads hit distinct
// banks) and kept in registers, permuted into the nibble-unpack order; the
// nibbles are multiplied as binary16 subnormals (pair_dot), then a DPP wave
// sum and an exact rescale by 2^20.
#include "common.hpp"
#include "q4_0.hpp"

namespace mote::q4_0 {
namespace {

constexpr int kStreamWaves = 8;
constexpr int kStreamThreads = kStreamWaves * kWave;
constexpr uint32_t kSlot = 144;
constexpr uint32_t kSubLo = 0x000F000Fu;  // low nibbles of bytes 0 and 2: n * 2^-24
constexpr uint32_t kSubHi = 0x00F000F0u;  // high nibbles of bytes 0 and 2: n * 2^-20
constexpr float kTwo20 = 1048576.0f;

__device__ __forceinline__ uint32_t pick(const uint32_t* x, int a, int b) {
    const uint32_t lo = (a & 1) ? 0x0302u : 0x0100u;
    const uint32_t hi = (b & 1) ? 0x07060000u : 0x05040000u;
    return __builtin_amdgcn_perm(x[b >> 1], x[a >> 1], hi | lo);
}

struct XPair {
    uint32_t xp[32];
    float c0, c1;  // -8 * 2^-20 * (sum of the block's 32 activations)
};

// sum_k x_k (n_k - 8) d of the two blocks of a pair, divided by 2^20.
//
// Nibbles are read as binary16 subnormals, with no carrier term and no shift
// for bytes 0 and 2 of a dword: q & 0x000F000F holds (n_b0, n_b2) * 2^-24 and
// q & 0x00F000F0 holds (n_b0, n_b2) * 2^-20 (the high nibbles); bytes 1 and 3
// take one shift by 8.  Each such value times an f16 activation is exact in
// f32 (v_dot2_f32_f16 honours f16 subnormals: the kernels run with f16
// denormals enabled), so per block
//   sum x (n - 8) = 2^20 (16 a_lo + a_hi)   with a_hi started at -8 * 2^-20 sum x,
// five VALU operations per nibble dword instead of a mask, shift and OR per
// nibble pair.
__device__ __forceinline__ float pair_dot(const uint32_t (&raw)[9], const XPair& x) {
    uint32_t q[8];
    q[0] = pair_q0(raw);
    q[1] = raw[1]; q[2] = raw[2]; q[3] = raw[3];
    q[4] = raw[5]; q[5] = raw[6]; q[6] = raw[7]; q[7] = raw[8];
    const float d0 = half_lo_to_float(raw[0]);
    const float d1 = half_hi_to_float(raw[4]);
    float lo0 = 0.0f, hi0 = x.c0, lo1 = 0.0f, hi1 = x.c1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t a = q[i], b = q[4 + i];
        const uint32_t a8 = a >> 8, b8 = b >> 8;
        hi0 = dot2(a & kSubHi, x.xp[4 * i + 0], hi0);
        lo0 = dot2(a & kSubLo, x.xp[4 * i + 1], lo0);
        lo0 = dot2(a8 & kSubLo, x.xp[4 * i + 2], lo0);
        hi0 = dot2(a8 & kSubHi, x.xp[4 * i + 3], hi0);
        hi1 = dot2(b & kSubHi, x.xp[16 + 4 * i + 0], hi1);
        lo1 = dot2(b & kSubLo, x.xp[16 + 4 * i + 1], lo1);
        lo1 = dot2(b8 & kSubLo, x.xp[16 + 4 * i + 2], lo1);
        hi1 = dot2(b8 & kSubHi, x.xp[16 + 4 * i + 3], hi1);
    }
    const float acc = d0 * __builtin_fmaf(lo0, 16.0f, hi0);
    return __builtin_fmaf(d1, __builtin_fmaf(lo1, 16.0f, hi1), acc);
}

template <int D, typename OutT>
__global__ __launch_bounds__(kStreamThreads) void gemv_stream_kernel(const uint16_t* __restrict__ x,
                                                                     const uint8_t* __restrict__ w,
                                                                     OutT* __restrict__ y, uint32_t N,
                                                                     uint32_t K, uint32_t total_waves) {
    extern __shared__ __attribute__((aligned(16))) uint8_t xs[];
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const uint32_t npairs = K >> 6;
    const size_t row_bytes = static_cast<size_t>(npairs) * kPairBytes;
    const uint32_t p = min(static_cast<uint32_t>(lane), npairs - 1);  // idle lanes: clamped, dropped
    const bool active = static_cast<uint32_t>(lane) < npairs;
    const uint32_t g = blockIdx.x * kStreamWaves + static_cast<uint32_t>(wave);
    // rows g, g + W, ...: count, and the last one (prefetches past it re-read
    // it, an L2 hit, so every load is unconditional and vmcnt stays exact)
    const uint32_t nrows = g < N ? (N - 1 - g) / total_waves + 1 : 0;
    const uint32_t last = g < N ? g + (nrows - 1) * total_waves : N - 1;
    const uint8_t* wl = w + static_cast<size_t>(p) * kPairBytes;

    // x chunk load first, then the first D rows.
    const uint32_t xchunks = npairs * 8;
    const uint32_t xc = min(static_cast<uint32_t>(tid), xchunks - 1);
    const u32x4 xreg = reinterpret_cast<const u32x4*>(x)[xc];
    __builtin_amdgcn_sched_barrier(0);
    uint32_t buf[D][9];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        const uint32_t r = min(g + static_cast<uint32_t>(d) * total_waves, last);
        load_pair(wl + static_cast<size_t>(r) * row_bytes, buf[d]);
    }
    *reinterpret_cast<u32x4*>(xs + (xc >> 3) * kSlot + (xc & 7) * 16) = xreg;
    __syncthreads();

    XPair xv;
    {
        uint32_t xr[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(xs + p * kSlot + i * 16);
            xr[4 * i + 0] = v.x; xr[4 * i + 1] = v.y; xr[4 * i + 2] = v.z; xr[4 * i + 3] = v.w;
        }
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            s0 = dot2(xr[i], kOnePair, s0);
            s1 = dot2(xr[16 + i], kOnePair, s1);
        }
        xv.c0 = (-8.0f / kTwo20) * s0;
        xv.c1 = (-8.0f / kTwo20) * s1;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int base = (q < 4) ? 0 : 32;
            const int e0 = base + pair_byte_element(q, 0);
            const int e1 = base + pair_byte_element(q, 1);
            const int e2 = base + pair_byte_element(q, 2);
            const int e3 = base + pair_byte_element(q, 3);
            xv.xp[4 * q + 0] = pick(xr, e0 + 16, e2 + 16);  // hi02
            xv.xp[4 * q + 1] = pick(xr, e0, e2);            // lo02
            xv.xp[4 * q + 2] = pick(xr, e1, e3);            // lo13
            xv.xp[4 * q + 3] = pick(xr, e1 + 16, e3 + 16);  // hi13
        }
    }

    // Row sums stay in registers (lane j % 64 holds row j of this wave) and
    // are stored every 64 rows and at the end, so no store sits between the
    // pipelined loads.  The loop runs at least once (a wave without rows
    // computes clamped rows and stores nothing), which keeps the first D
    // loads ahead of the x barrier.
    float mine = 0.0f;
    uint32_t j = 0;
    do {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const uint32_t jj = j + static_cast<uint32_t>(d);
            const float s = wave_sum(active ? pair_dot(buf[d], xv) : 0.0f);
            mine = (jj < nrows && static_cast<uint32_t>(lane) == (jj & 63u)) ? s : mine;
            const uint32_t r = min(g + (jj + D) * total_waves, last);
            load_pair(wl + static_cast<size_t>(r) * row_bytes, buf[d]);
            if ((jj & 63u) == 63u && jj < nrows) {  // uniform: flush a full slot set
                y[g + (jj - 63u + static_cast<uint32_t>(lane)) * total_waves] = to_out<OutT>(kTwo20 * mine);
            }
        }
        j += D;
    } while (j < nrows);
    const uint32_t base = nrows & ~63u;
    if (static_cast<uint32_t>(lane) < nrows - base)
        y[g + (base + static_cast<uint32_t>(lane)) * total_waves] = to_out<OutT>(kTwo20 * mine);
}

template <int D, int G>
hipError_t launch_gemv_stream(const Problem& p) {
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        return n;
    }();
    uint32_t groups = static_cast<uint32_t>(cus) * G;
    const uint32_t need = (p.N + kStreamWaves - 1) / kStreamWaves;  // no idle workgroups
    if (groups > need) groups = need;
    const uint32_t total_waves = groups * kStreamWaves;
    const size_t lds = static_cast<size_t>(p.K / 64) * kSlot;
    const dim3 grid(groups), block(kStreamThreads);
    if (p.out == OutType::F32) {
        hipLaunchKernelGGL((gemv_stream_kernel<D, float>), grid, block, lds, p.stream,
                           static_cast<const uint16_t*>(p.x), static_cast<const uint8_t*>(p.w),
                           static_cast<float*>(p.y), p.N, p.K, total_waves);
    } else {
        hipLaunchKernelGGL((gemv_stream_kernel<D, _Float16>), grid, block, lds, p.stream,
                           static_cast<const uint16_t*>(p.x), static_cast<const uint8_t*>(p.w),
                           static_cast<_Float16*>(p.y), p.N, p.K, total_waves);
    }
    return hipGetLastError();
}

#define MOTE_STREAM(D, G) \
    Variant{"stream_d" #D "_g" #G, Kind::GemvStream, D, G, 1, &launch_gemv_stream<D, G>}

const Variant kStream[] = {
    MOTE_STREAM(1, 1), MOTE_STREAM(2, 1), MOTE_STREAM(3, 1), MOTE_STREAM(4, 1),
    MOTE_STREAM(1, 2), MOTE_STREAM(2, 2), MOTE_STREAM(3, 2), MOTE_STREAM(4, 2),
    MOTE_STREAM(2, 3), MOTE_STREAM(2, 4),
};

#undef MOTE_STREAM

}  // namespace

const Variant* gemv_stream_variants(int* count) {
    *count = static_cast<int>(sizeof(kStream) / sizeof(kStream[0]));
    return kStream;
}

// One token, K a multiple of 64 and at most 4096 (one pair per lane), x 16-byte
// and w dword aligned.
bool gemv_stream_supports(const Variant& v, const Problem& p) {
    (void)v;
    return p.M == 1 && p.K % 64 == 0 && p.K > 0 && p.K <= 4096 &&
           reinterpret_cast<uintptr_t>(p.w) % 4 == 0 && reinterpret_cast<uintptr_t>(p.x) % 16 == 0;
}

}  // namespace mote::q4_0

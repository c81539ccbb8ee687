// Q4_0 decode GEMV (M = 1) for gfx950: row-streaming waves with the
// activation vector staged once per workgroup in LDS.
//
// Computes y[n] = sum_k x[k] * w[n, k] for f16 x [K] and GGML Q4_0 w [N, K],
// the operation of crates/mote-backend-hip/src/quantized_linear.hip:13-52
// (oracle crates/mote-reference/src/quantized.rs:89-144) at rows == 1.
//
// Mapping (one 512-thread workgroup = 8 waves):
//  * K is cut into 64-element block pairs (36 bytes, dword aligned); lane l of
//    K-slice wave kg owns pair p = 64 kg + l of every row, so KS waves cover a
//    row of up to 64 KS pairs (K <= 4096 KS) and the 8 / KS wave groups of the
//    workgroup take R consecutive rows each;
//  * every thread issues its coalesced 16-byte loads of x and then the loads
//    of its R pairs (R x 9 dwords; plain loads: non-temporal ones measured
//    slower for this dword-aligned pattern); x goes to LDS, one 128-byte pair chunk per 144-byte slot, so the 8
//    chunk reads of the 64 lanes of a wave (stride 36 dwords) fall on
//    distinct banks;
//  * each lane keeps its pair of x in registers, permuted once into the order
//    the nibble unpack produces (the same scheme as the skinny kernel: 1 + n/64
//    binary16 values, v_dot2_f32_f16, minus 1.125 sum(x), times the scale), so
//    the R rows of a wave reuse it and cost only their own loads and ALU;
//  * rows are summed across the wave with DPP and, for KS > 1, across the K
//    slices through LDS in a fixed order (deterministic), then scaled by 64.
//
// Workgroup b runs on XCD b % 8; tile (b % 8) * per_xcd + b / 8 gives each XCD
// a contiguous run of rows.
#include "common.hpp"
#include "gemv_formats.hpp"
#include "q4_0.hpp"

namespace mote::q4_0 {
namespace {

constexpr int kRowsWaves = 8;
constexpr int kRowsThreads = kRowsWaves * kWave;
constexpr uint32_t kChunkSlot = 144;  // bytes of LDS per 128-byte pair chunk of x

template <int R, int KS, typename OutT>
__global__ __launch_bounds__(kRowsThreads) void gemv_rows_kernel(const uint16_t* __restrict__ x,
                                                                 const uint8_t* __restrict__ w,
                                                                 OutT* __restrict__ y, uint32_t N,
                                                                 uint32_t K, uint32_t total,
                                                                 uint32_t per_xcd) {
    constexpr int RG = kRowsWaves / KS;
    extern __shared__ __attribute__((aligned(16))) uint8_t xs[];
    __shared__ float partial[KS > 1 ? kRowsWaves * R : 1];

    const int tid = static_cast<int>(threadIdx.x);
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int kg = wave % KS;
    const int rg = wave / KS;
    const uint32_t one = one_pair_reg();  // binary16 (1, 1): one v_and_or_b32 per nibble pair

    const uint32_t tile = (blockIdx.x % 8u) * per_xcd + blockIdx.x / 8u;
    if (tile >= total) return;  // uniform for the workgroup, before any barrier
    const uint32_t row0 = (tile * RG + rg) * R;
    const uint32_t npairs = K >> 6;
    const size_t row_bytes = static_cast<size_t>(npairs) * kPairBytes;
    const uint32_t p = static_cast<uint32_t>(kg * kWave + lane);
    const bool active = p < npairs;
    const uint32_t pc = min(p, npairs - 1);  // idle lanes load a valid pair and drop it
    const uint32_t xchunks = npairs * 8;

    // 1. The x chunks first, then the weight stream.  vmcnt counts loads in
    //    issue order, so staging x waits only for x, and row r below waits
    //    only for rows 0..r.  No load is predicated (clamped addresses), which
    //    keeps the counts exact.
    u32x4 xreg[KS];
    const u32x4* xv = reinterpret_cast<const u32x4*>(x);
    uint32_t xc[KS];
#pragma unroll
    for (int j = 0; j < KS; ++j) {
        xc[j] = min(static_cast<uint32_t>(tid + kRowsThreads * j), xchunks - 1);
        xreg[j] = xv[xc[j]];
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the x loads ahead of the weight loads
    uint32_t raw[R][9];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t n = min(row0 + r, N - 1);
        load_pair(w + static_cast<size_t>(n) * row_bytes + static_cast<size_t>(pc) * kPairBytes, raw[r]);
    }

    // 2. Stage x in LDS: 8 chunks per pair, one 144-byte slot per pair (a
    //    clamped duplicate writes the same bytes to the same slot).
#pragma unroll
    for (int j = 0; j < KS; ++j)
        *reinterpret_cast<u32x4*>(xs + (xc[j] >> 3) * kChunkSlot + (xc[j] & 7) * 16) = xreg[j];
    __syncthreads();

    // 3. This lane's 64 activations, permuted into unpack order (idle lanes
    //    read the clamped pair; their sums are dropped below).
    uint32_t xp[32];
    float c0, c1;
    {
        uint32_t xr[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(xs + pc * kChunkSlot + i * 16);
            xr[4 * i + 0] = v.x; xr[4 * i + 1] = v.y; xr[4 * i + 2] = v.z; xr[4 * i + 3] = v.w;
        }
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            s0 = dot2(xr[i], kOnePair, s0);
            s1 = dot2(xr[16 + i], kOnePair, s1);
        }
        c0 = -1.125f * s0;
        c1 = -1.125f * s1;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int base = (q < 4) ? 0 : 32;
            const int e0 = base + pair_byte_element(q, 0);
            const int e1 = base + pair_byte_element(q, 1);
            const int e2 = base + pair_byte_element(q, 2);
            const int e3 = base + pair_byte_element(q, 3);
            xp[4 * q + 0] = pick(xr, e0 + 16, e2 + 16);  // hi02
            xp[4 * q + 1] = pick(xr, e0, e2);            // lo02
            xp[4 * q + 2] = pick(xr, e1, e3);            // lo13
            xp[4 * q + 3] = pick(xr, e1 + 16, e3 + 16);  // hi13
        }
    }

    // 4. Dot products, row by row in load order.
    float sums[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        uint32_t q[8];
        q[0] = pair_q0(raw[r]);
        q[1] = raw[r][1]; q[2] = raw[r][2]; q[3] = raw[r][3];
        q[4] = raw[r][5]; q[5] = raw[r][6]; q[6] = raw[r][7]; q[7] = raw[r][8];
        const float d0 = half_lo_to_float(raw[r][0]);
        const float d1 = half_hi_to_float(raw[r][4]);
        float a0 = c0, a1 = c1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a0 = dot2(nib_hi02(q[i], one), xp[4 * i + 0], a0);
            a0 = dot2(nib_lo02(q[i], one), xp[4 * i + 1], a0);
            a0 = dot2(nib_lo13(q[i], one), xp[4 * i + 2], a0);
            a0 = dot2(nib_hi13(q[i], one), xp[4 * i + 3], a0);
            a1 = dot2(nib_hi02(q[4 + i], one), xp[16 + 4 * i + 0], a1);
            a1 = dot2(nib_lo02(q[4 + i], one), xp[16 + 4 * i + 1], a1);
            a1 = dot2(nib_lo13(q[4 + i], one), xp[16 + 4 * i + 2], a1);
            a1 = dot2(nib_hi13(q[4 + i], one), xp[16 + 4 * i + 3], a1);
        }
        float acc = __builtin_fmaf(d0, a0, 0.0f);
        acc = __builtin_fmaf(d1, a1, acc);
        float s = wave_sum(active ? acc : 0.0f);
        // A sum that is not finite (an infinite scale or a non-finite
        // activation): the wave's share of the row again with the reference's
        // per-element arithmetic (gemv_formats.hpp).  Wave-uniform.
        if (__builtin_expect(not_finite(s), 0)) {
            const uint8_t* pair = w + static_cast<size_t>(min(row0 + r, N - 1)) * row_bytes +
                                  static_cast<size_t>(pc) * kPairBytes;
            const float e = active ? q4_0_exact_pair(pair, x + static_cast<size_t>(pc) * 64) : 0.0f;
            s = wave_sum(e) * (1.0f / 64.0f);
        }
        sums[r] = s;
    }

    float mine = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) mine = (lane == r) ? sums[r] : mine;

    if constexpr (KS > 1) {
        if (lane < R) partial[wave * R + lane] = mine;
        __syncthreads();
        if (kg != 0) return;
        if (lane < R) {
            float s = partial[wave * R + lane];
#pragma unroll
            for (int k = 1; k < KS; ++k) s += partial[(wave + k) * R + lane];
            mine = s;
        }
    }
    if (lane < R) {
        const uint32_t n = row0 + static_cast<uint32_t>(lane);
        if (n < N) y[n] = to_out<OutT>(64.0f * mine);
    }
}

template <int R, int KS>
hipError_t launch_gemv_rows(const Problem& p) {
    constexpr int RG = kRowsWaves / KS;
    const uint32_t rows_per_wg = RG * R;
    const uint32_t total = (p.N + rows_per_wg - 1) / rows_per_wg;
    const uint32_t per_xcd = (total + 7u) / 8u;
    const size_t lds = static_cast<size_t>(p.K / 64) * kChunkSlot;
    const dim3 grid(per_xcd * 8u), block(kRowsThreads);
    if (p.out == OutType::F32) {
        hipLaunchKernelGGL((gemv_rows_kernel<R, KS, float>), grid, block, lds, p.stream,
                           static_cast<const uint16_t*>(p.x), static_cast<const uint8_t*>(p.w),
                           static_cast<float*>(p.y), p.N, p.K, total, per_xcd);
    } else {
        hipLaunchKernelGGL((gemv_rows_kernel<R, KS, _Float16>), grid, block, lds, p.stream,
                           static_cast<const uint16_t*>(p.x), static_cast<const uint8_t*>(p.w),
                           static_cast<_Float16*>(p.y), p.N, p.K, total, per_xcd);
    }
    return hipGetLastError();
}

#define MOTE_ROWS(R, KS) \
    Variant{"rows_r" #R "_k" #KS, Kind::GemvRows, R, 1, KS, &launch_gemv_rows<R, KS>}

const Variant kRows[] = {
    MOTE_ROWS(4, 1), MOTE_ROWS(4, 2), MOTE_ROWS(4, 4), MOTE_ROWS(4, 8),
};

#undef MOTE_ROWS

}  // namespace

const Variant* gemv_rows_variants(int* count) {
    *count = static_cast<int>(sizeof(kRows) / sizeof(kRows[0]));
    return kRows;
}

// One token, K a multiple of 64 that one row of KS waves covers and whose x
// fits the 64 KB of LDS a workgroup may allocate, x 16-byte and w dword
// aligned.
bool gemv_rows_supports(const Variant& v, const Problem& p) {
    const uint32_t ks = static_cast<uint32_t>(v.p2);
    const uint64_t lds = static_cast<uint64_t>(p.K / 64) * kChunkSlot;
    return p.M == 1 && p.K % 64 == 0 && p.K > 0 && p.K <= 4096u * ks && lds <= 65536 &&
           reinterpret_cast<uintptr_t>(p.w) % 4 == 0 && reinterpret_cast<uintptr_t>(p.x) % 16 == 0;
}

}  // namespace mote::q4_0

// Q4_0 decode GEMV and skinny GEMM on the vector ALUs (M <= 63).
//
// Computes y[m, n] = sum_k x[m, k] * w[n, k] for f16 activations x [M, K] and
// GGML Q4_0 weights w [N, K], the operation of
// crates/mote-backend-hip/src/quantized_linear.hip:13-52 with the oracle
// crates/mote-reference/src/quantized.rs:89-144.
//
// Mapping (one 256-thread workgroup = 4 waves):
//  * a lane owns one 36-byte block pair (64 elements of K) per step and walks
//    the pairs p = lane, lane + 64*KSPLIT, ...; KSPLIT waves of the workgroup
//    split K between them and meet in LDS at the end;
//  * a wave owns R consecutive weight rows and MT consecutive tokens, so each
//    lane issues R pair loads (9 dwords each) before any arithmetic and keeps
//    the activations for its pair in registers, permuted once into the order
//    the nibble unpack produces them and reused by all R rows;
//  * per block: 16 v_dot2_f32_f16 on (1 + n/64) * x, started from
//    -1.125 * sum(x), then one FMA with the block scale: sum (n - 8) x d / 64;
//  * rows are reduced across the wave with DPP and across the KSPLIT waves
//    through LDS; the final factor 64 is an exact power-of-two rescale.
//
// Workgroups are mapped XCD-aware: the hardware deals workgroup b to XCD
// b % 8, so logical tile (b % 8) * per_xcd + b / 8 gives each XCD a contiguous
// run of tiles, and the token chunks of one row tile share that XCD's L2.
#include "common.hpp"
#include "gemv_formats.hpp"
#include "q4_0.hpp"

namespace mote::q4_0 {
namespace {

__device__ __forceinline__ uint32_t pick_rt(const uint32_t* x, int a, int b) {
    const uint32_t lo = (a & 1) ? 0x0302u : 0x0100u;
    const uint32_t hi = (b & 1) ? 0x07060000u : 0x05040000u;
    return __builtin_amdgcn_perm(x[b >> 1], x[a >> 1], hi | lo);
}

template <int R, int MT, int KSPLIT, typename OutT>
__global__ __launch_bounds__(256) void gemv_kernel(const uint16_t* __restrict__ x,
                                                   const uint8_t* __restrict__ w,
                                                   OutT* __restrict__ y, uint32_t M,
                                                   uint32_t N, uint32_t K,
                                                   uint32_t token_chunks, uint32_t total,
                                                   uint32_t per_xcd) {
    constexpr int RG = 4 / KSPLIT;
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int kg = wave % KSPLIT;
    const int rg = wave / KSPLIT;
    const uint32_t one = one_pair_reg();  // binary16 (1, 1): one v_and_or_b32 per nibble pair

    const uint32_t logical = (blockIdx.x % 8u) * per_xcd + blockIdx.x / 8u;
    if (logical >= total) return;  // uniform for the workgroup, before any barrier
    const uint32_t tile = logical / token_chunks;
    const uint32_t tc = logical - tile * token_chunks;
    const uint32_t row0 = (tile * RG + rg) * R;
    const uint32_t t0 = tc * MT;
    const uint32_t npairs = K >> 6;
    const size_t row_bytes = static_cast<size_t>(npairs) * kPairBytes;

    const uint8_t* wrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t n = min(row0 + r, N - 1);
        wrow[r] = w + static_cast<size_t>(n) * row_bytes;
    }
    const uint16_t* xrow[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const uint32_t m = min(t0 + t, M - 1);
        xrow[t] = x + static_cast<size_t>(m) * K;
    }

    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[r][t] = 0.0f;

    for (uint32_t p = kg * kWave + lane; p < npairs; p += kWave * KSPLIT) {
        uint32_t raw[R][9];
#pragma unroll
        for (int r = 0; r < R; ++r) load_pair(wrow[r] + static_cast<size_t>(p) * kPairBytes, raw[r]);

        uint32_t xp[MT][32];
        float c0[MT], c1[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            uint32_t xr[32];
            const u32x4* src = reinterpret_cast<const u32x4*>(xrow[t] + static_cast<size_t>(p) * 64);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const u32x4 v = src[i];
                xr[4 * i + 0] = v.x; xr[4 * i + 1] = v.y; xr[4 * i + 2] = v.z; xr[4 * i + 3] = v.w;
            }
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                s0 = dot2(xr[i], kOnePair, s0);
                s1 = dot2(xr[16 + i], kOnePair, s1);
            }
            c0[t] = -1.125f * s0;
            c1[t] = -1.125f * s1;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int base = (q < 4) ? 0 : 32;
                const int e0 = base + pair_byte_element(q, 0);
                const int e1 = base + pair_byte_element(q, 1);
                const int e2 = base + pair_byte_element(q, 2);
                const int e3 = base + pair_byte_element(q, 3);
                xp[t][4 * q + 0] = pick_rt(xr, e0 + 16, e2 + 16);  // hi02
                xp[t][4 * q + 1] = pick_rt(xr, e0, e2);            // lo02
                xp[t][4 * q + 2] = pick_rt(xr, e1, e3);            // lo13
                xp[t][4 * q + 3] = pick_rt(xr, e1 + 16, e3 + 16);  // hi13
            }
        }

#pragma unroll
        for (int r = 0; r < R; ++r) {
            uint32_t q[8];
            q[0] = pair_q0(raw[r]);
            q[1] = raw[r][1]; q[2] = raw[r][2]; q[3] = raw[r][3];
            q[4] = raw[r][5]; q[5] = raw[r][6]; q[6] = raw[r][7]; q[7] = raw[r][8];
            const float d0 = half_lo_to_float(raw[r][0]);
            const float d1 = half_hi_to_float(raw[r][4]);
            uint32_t u[32];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                u[4 * i + 0] = nib_hi02(q[i], one);
                u[4 * i + 1] = nib_lo02(q[i], one);
                u[4 * i + 2] = nib_lo13(q[i], one);
                u[4 * i + 3] = nib_hi13(q[i], one);
            }
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                float a0 = c0[t], a1 = c1[t];
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    a0 = dot2(u[i], xp[t][i], a0);
                    a1 = dot2(u[16 + i], xp[t][16 + i], a1);
                }
                acc[r][t] = __builtin_fmaf(d0, a0, acc[r][t]);
                acc[r][t] = __builtin_fmaf(d1, a1, acc[r][t]);
            }
        }
    }

    // Wave reduction: every lane ends up holding all R*MT sums.
    float sums[R * MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            float s = wave_sum(acc[r][t]);
            // A sum that is not finite (an infinite scale or a non-finite
            // activation): this wave's share of the row again with the
            // reference's per-element arithmetic (gemv_formats.hpp), in the
            // units of the dot chains.  Wave-uniform; ordinary rows skip it.
            if (__builtin_expect(not_finite(s), 0)) {
                float e = 0.0f;
                for (uint32_t p = kg * kWave + lane; p < npairs; p += kWave * KSPLIT)
                    e += q4_0_exact_pair(wrow[r] + static_cast<size_t>(p) * kPairBytes,
                                         xrow[t] + static_cast<size_t>(p) * 64);
                s = wave_sum(e) * (1.0f / 64.0f);
            }
            sums[t * R + r] = s;
        }

    float mine = 0.0f;
#pragma unroll
    for (int i = 0; i < R * MT; ++i) mine = (lane == i) ? sums[i] : mine;

    if constexpr (KSPLIT > 1) {
        __shared__ float partial[4][R * MT];
        if (lane < R * MT) partial[wave][lane] = mine;
        __syncthreads();
        if (kg != 0) return;
        if (lane < R * MT) {
            float s = partial[wave][lane];
#pragma unroll
            for (int k = 1; k < KSPLIT; ++k) s += partial[wave + k][lane];
            mine = s;
        }
    }
    if (lane < R * MT) {
        const uint32_t r = static_cast<uint32_t>(lane) % R;
        const uint32_t t = static_cast<uint32_t>(lane) / R;
        const uint32_t n = row0 + r;
        const uint32_t m = t0 + t;
        if (n < N && m < M) y[static_cast<size_t>(m) * N + n] = to_out<OutT>(64.0f * mine);
    }
}

template <int R, int MT, int KSPLIT>
hipError_t launch_gemv(const Problem& p) {
    constexpr int RG = 4 / KSPLIT;
    const uint32_t rows_per_wg = RG * R;
    const uint32_t row_tiles = (p.N + rows_per_wg - 1) / rows_per_wg;
    const uint32_t token_chunks = (p.M + MT - 1) / MT;
    const uint64_t total64 = static_cast<uint64_t>(row_tiles) * token_chunks;
    if (total64 > 0x7fffffffull) return hipErrorInvalidConfiguration;
    const uint32_t total = static_cast<uint32_t>(total64);
    const uint32_t per_xcd = (total + 7u) / 8u;
    const dim3 grid(per_xcd * 8u), block(256);
    if (p.out == OutType::F32) {
        hipLaunchKernelGGL((gemv_kernel<R, MT, KSPLIT, float>), grid, block, 0, p.stream,
                           static_cast<const uint16_t*>(p.x), static_cast<const uint8_t*>(p.w),
                           static_cast<float*>(p.y), p.M, p.N, p.K, token_chunks, total, per_xcd);
    } else {
        hipLaunchKernelGGL((gemv_kernel<R, MT, KSPLIT, _Float16>), grid, block, 0, p.stream,
                           static_cast<const uint16_t*>(p.x), static_cast<const uint8_t*>(p.w),
                           static_cast<_Float16*>(p.y), p.M, p.N, p.K, token_chunks, total,
                           per_xcd);
    }
    return hipGetLastError();
}

#define MOTE_GEMV(R, MT, KS) \
    Variant{"gemv_r" #R "_t" #MT "_k" #KS, Kind::Gemv, R, MT, KS, &launch_gemv<R, MT, KS>}

// The shapes the dispatch heuristic falls back to (M = 1 beyond the
// streaming GEMV's K range, 2-63 tokens where no matrix-core tiling fits).
const Variant kGemv[] = {
    MOTE_GEMV(4, 1, 1), MOTE_GEMV(2, 1, 1), MOTE_GEMV(4, 1, 2), MOTE_GEMV(4, 2, 1), MOTE_GEMV(4, 4, 1),
};

#undef MOTE_GEMV

}  // namespace

const Variant* gemv_variants(int* count) {
    *count = static_cast<int>(sizeof(kGemv) / sizeof(kGemv[0]));
    return kGemv;
}

bool gemv_supports(const Variant& v, const Problem& p) {
    (void)v;
    return p.K % 64 == 0 && p.K > 0 &&
           reinterpret_cast<uintptr_t>(p.w) % 4 == 0 &&
           reinterpret_cast<uintptr_t>(p.x) % 16 == 0;
}

}  // namespace mote::q4_0

// Q4_0 prefill-shaped linear (M >= 64) on the CDNA4 matrix cores, plus the
// fused gate/up SiLU-mul variant.
//
//   y[m, n] = sum_k x[m, k] * w[n, k]                                (linear)
//   y[m, n] = silu(sum_k x w_gate[n, k]) * (sum_k x w_up[n, k])       (gate/up)
//
// The linear is the operation of crates/mote-backend-hip/src/
// quantized_linear.hip:13-52 (oracle crates/mote-reference/src/quantized.rs:
// 89-144); the fused gate/up has no counterpart in the reference.
//
// One 256-thread workgroup computes a BM x BN output tile with 2 x 2 waves,
// each wave a (BM/2) x (BN/2) grid of 16x16 v_mfma_f32_16x16x32_f16 tiles.
// K advances 64 elements (one Q4_0 block pair per weight row) per step through
// a double-buffered LDS stage:
//  * activations: BM rows x 64 f16 copied from HBM, stored in the k order the
//    weight dequantisation produces (below);
//  * weights: BN rows x 36 bytes loaded as dwords, dequantised in registers to
//    f16 (q - 8) * d  (exact q - 8 from the 1024 + q exponent-bias trick, one
//    binary16 rounding for the product) and stored to LDS.
// A 32-element block is split into four k groups g = 0..3: nibble bytes
// 4g..4g+3, i.e. elements {4g..4g+3} and {16+4g..16+4g+3}, each stored as
// [4g, 4g+2, 4g+1, 4g+3, 16+4g, 16+4g+2, 16+4g+1, 16+4g+3].  MFMA lane group g
// (lanes 16g..16g+15) reads group g of both operands, so A and B agree on k.
// LDS rows are padded to 144 bytes so the 16 rows read by one MFMA operand
// fall on distinct banks.
#include "common.hpp"
#include "q4_0.hpp"

namespace mote::q4_0 {
namespace {

constexpr int kRowHalves = 72;  // 64 halves + 8 halves padding per LDS row
constexpr int kRowBytes = kRowHalves * 2;

// Dequantises the four k groups of one block.  `g[i]` holds nibble bytes
// 4i..4i+3 of the block, `scale` the block's f16 scale bits in its low half.
__device__ __forceinline__ void dequant_block(const uint32_t (&g)[4], uint32_t scale,
                                              u32x4 (&out)[4]) {
    const f16x2 dd = as_h2(__builtin_amdgcn_perm(scale, scale, 0x01000100u));
    const f16x2 bias = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t q = g[i];
        const uint32_t lo02 = (q & 0x000F000Fu) | 0x64006400u;
        const uint32_t lo13 = ((q >> 8) & 0x000F000Fu) | 0x64006400u;
        const uint32_t hi02 = ((q >> 4) & 0x000F000Fu) | 0x64006400u;
        const uint32_t hi13 = ((q >> 12) & 0x000F000Fu) | 0x64006400u;
        out[i].x = __builtin_bit_cast(uint32_t, (as_h2(lo02) + bias) * dd);
        out[i].y = __builtin_bit_cast(uint32_t, (as_h2(lo13) + bias) * dd);
        out[i].z = __builtin_bit_cast(uint32_t, (as_h2(hi02) + bias) * dd);
        out[i].w = __builtin_bit_cast(uint32_t, (as_h2(hi13) + bias) * dd);
    }
}

template <int BM, int BN>
struct Tile {
    static constexpr int kXChunks = BM * 8 / 256;          // 16-byte x chunks per thread
    static constexpr int kWItems = (BN * 2 + 255) / 256;   // (row, block) items per thread
};

// Loads one block of weight row `n` at k-pair `kp`: five dwords covering the
// block's scale and nibbles.
__device__ __forceinline__ void load_block(const uint8_t* pair, int blk, uint32_t (&d)[5]) {
    if (blk == 0) {
        const u32x4_a4 a = *reinterpret_cast<const u32x4_a4*>(pair);
        d[0] = a.x; d[1] = a.y; d[2] = a.z; d[3] = a.w;
        d[4] = *reinterpret_cast<const uint32_t*>(pair + 16);
    } else {
        d[0] = *reinterpret_cast<const uint32_t*>(pair + 16);
        const u32x4_a4 a = *reinterpret_cast<const u32x4_a4*>(pair + 20);
        d[1] = a.x; d[2] = a.y; d[3] = a.z; d[4] = a.w;
    }
}

// Groups and scale of a loaded block (see load_block).
__device__ __forceinline__ void block_groups(const uint32_t (&d)[5], int blk, uint32_t (&g)[4],
                                             uint32_t& scale) {
    if (blk == 0) {
        scale = d[0];
        g[0] = __builtin_amdgcn_perm(d[1], d[0], 0x05040302u);
        g[1] = __builtin_amdgcn_perm(d[2], d[1], 0x05040302u);
        g[2] = __builtin_amdgcn_perm(d[3], d[2], 0x05040302u);
        g[3] = __builtin_amdgcn_perm(d[4], d[3], 0x05040302u);
    } else {
        scale = d[0] >> 16;
        g[0] = d[1]; g[1] = d[2]; g[2] = d[3]; g[3] = d[4];
    }
}

template <int BM, int BN, bool GATE_UP, int PF, typename OutT>
__global__ __launch_bounds__(256) void mfma_kernel(const uint16_t* __restrict__ x,
                                                   const uint8_t* __restrict__ wg,
                                                   const uint8_t* __restrict__ wu,
                                                   OutT* __restrict__ y, uint32_t M, uint32_t N,
                                                   uint32_t K, uint32_t m_tiles, uint32_t total,
                                                   uint32_t per_xcd) {
    using T = Tile<BM, BN>;
    constexpr int TM = BM / 32;  // 16-row MFMA tiles per wave along M
    constexpr int TN = BN / 32;  // along N
    constexpr int NW = GATE_UP ? 2 : 1;

    __shared__ __attribute__((aligned(16))) uint8_t xs[2][BM * kRowBytes];
    __shared__ __attribute__((aligned(16))) uint8_t ws[NW][2][BN * kRowBytes];

    const uint32_t logical = (blockIdx.x % 8u) * per_xcd + blockIdx.x / 8u;
    if (logical >= total) return;
    const uint32_t tile_n = logical / m_tiles;
    const uint32_t tile_m = logical - tile_n * m_tiles;
    const uint32_t m0 = tile_m * BM;
    const uint32_t n0 = tile_n * BN;

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const uint32_t npairs = K >> 6;
    const size_t row_bytes = static_cast<size_t>(npairs) * kPairBytes;
    const uint8_t* wsrc[NW] = {wg};
    if constexpr (GATE_UP) wsrc[1] = wu;

    // Per-thread load assignments.
    const uint16_t* xptr[T::kXChunks];
    int xoff[T::kXChunks][2];
#pragma unroll
    for (int j = 0; j < T::kXChunks; ++j) {
        const int c = tid + 256 * j;
        const int row = c >> 3, chunk = c & 7;
        const uint32_t m = min(m0 + row, M - 1);
        xptr[j] = x + static_cast<size_t>(m) * K + chunk * 8;
        const int blk = chunk >> 2, kin = (chunk & 3) * 8;
        const int half = kin >= 16 ? 1 : 0;
        const int g0 = (kin & 15) >> 2;
        xoff[j][0] = row * kRowBytes + blk * 64 + g0 * 16 + half * 8;
        xoff[j][1] = xoff[j][0] + 16;
    }
    const uint8_t* wptr[NW][T::kWItems];
    int woff[T::kWItems], wblk[T::kWItems];
    bool wlive[T::kWItems];
#pragma unroll
    for (int j = 0; j < T::kWItems; ++j) {
        const int item = tid + 256 * j;
        wlive[j] = item < BN * 2;
        const int row = wlive[j] ? item >> 1 : 0;
        wblk[j] = item & 1;
        const uint32_t n = min(n0 + row, N - 1);
#pragma unroll
        for (int s = 0; s < NW; ++s) wptr[s][j] = wsrc[s] + static_cast<size_t>(n) * row_bytes;
        woff[j] = row * kRowBytes + wblk[j] * 64;
    }

    // A ring of PF register stages: the global loads of step k are issued PF
    // steps before step k is written to LDS, so their HBM latency hides
    // behind PF steps of matrix-core work.  Steps past the end are clamped
    // to the last one (a re-read), which keeps every load unconditional and
    // the wait counts exact.
    u32x4 xreg[PF][T::kXChunks];
    uint32_t wreg[PF][NW][T::kWItems][5];

    auto load_stage = [&](uint32_t kp, int r) {
        kp = min(kp, npairs - 1);
#pragma unroll
        for (int j = 0; j < T::kXChunks; ++j)
            xreg[r][j] = *reinterpret_cast<const u32x4*>(xptr[j] + static_cast<size_t>(kp) * 64);
#pragma unroll
        for (int s = 0; s < NW; ++s)
#pragma unroll
            for (int j = 0; j < T::kWItems; ++j)
                if (wlive[j]) load_block(wptr[s][j] + static_cast<size_t>(kp) * kPairBytes, wblk[j], wreg[r][s][j]);
    };
    auto store_stage = [&](int buf, int r) {
#pragma unroll
        for (int j = 0; j < T::kXChunks; ++j) {
            const u32x4 v = xreg[r][j];
            u32x2 a, b;
            a.x = __builtin_amdgcn_perm(v.y, v.x, 0x05040100u);  // (x0, x2)
            a.y = __builtin_amdgcn_perm(v.y, v.x, 0x07060302u);  // (x1, x3)
            b.x = __builtin_amdgcn_perm(v.w, v.z, 0x05040100u);  // (x4, x6)
            b.y = __builtin_amdgcn_perm(v.w, v.z, 0x07060302u);  // (x5, x7)
            *reinterpret_cast<u32x2*>(&xs[buf][xoff[j][0]]) = a;
            *reinterpret_cast<u32x2*>(&xs[buf][xoff[j][1]]) = b;
        }
#pragma unroll
        for (int s = 0; s < NW; ++s)
#pragma unroll
            for (int j = 0; j < T::kWItems; ++j) {
                if (!wlive[j]) continue;
                uint32_t g[4], scale;
                block_groups(wreg[r][s][j], wblk[j], g, scale);
                u32x4 out[4];
                dequant_block(g, scale, out);
                u32x4* dst = reinterpret_cast<u32x4*>(&ws[s][buf][woff[j]]);
                dst[0] = out[0]; dst[1] = out[1]; dst[2] = out[2]; dst[3] = out[3];
            }
    };

    f32x4 acc[NW][TM][TN];
#pragma unroll
    for (int s = 0; s < NW; ++s)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[s][i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int lrow = lane & 15;
    const int lgrp = lane >> 4;
    const int a_base = (wm * (BM / 2) + lrow) * kRowBytes + lgrp * 16;
    const int b_base = (wn * (BN / 2) + lrow) * kRowBytes + lgrp * 16;

    auto mma_step = [&](int buf) {
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            f16x8 a[TM];
#pragma unroll
            for (int i = 0; i < TM; ++i)
                a[i] = *reinterpret_cast<const f16x8*>(&xs[buf][a_base + i * 16 * kRowBytes + blk * 64]);
#pragma unroll
            for (int s = 0; s < NW; ++s) {
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const f16x8 b =
                        *reinterpret_cast<const f16x8*>(&ws[s][buf][b_base + j * 16 * kRowBytes + blk * 64]);
#pragma unroll
                    for (int i = 0; i < TM; ++i)
                        acc[s][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b, acc[s][i][j], 0, 0, 0);
                }
            }
        }
    };

    // Prologue: steps 0 .. PF-1 in flight, step 0 in LDS, step PF loading.
#pragma unroll
    for (int r = 0; r < PF; ++r) load_stage(static_cast<uint32_t>(r), r);
    store_stage(0, 0);
    load_stage(PF, 0);
    __syncthreads();

    // Iteration k: write step k + 1 (ring slot (k + 1) % PF) to the other LDS
    // buffer, refill that slot with step k + 1 + PF, multiply step k.  The
    // loop is unrolled by PF so ring slots are compile-time constants.
    for (uint32_t kp = 0; kp < npairs; kp += PF) {
#pragma unroll
        for (int d = 0; d < PF; ++d) {
            const uint32_t k = kp + static_cast<uint32_t>(d);
            if (k < npairs) {  // uniform
                const int buf = static_cast<int>(k & 1u);
                const int slot = (d + 1) % PF;
                if (k + 1 < npairs) {
                    store_stage(buf ^ 1, slot);
                    load_stage(k + 1 + PF, slot);
                }
                mma_step(buf);
                __syncthreads();
            }
        }
    }

    // Epilogue: lane holds rows 4*lgrp .. 4*lgrp+3, column lrow of each tile.
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint32_t n = n0 + wn * (BN / 2) + j * 16 + lrow;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t m = m0 + wm * (BM / 2) + i * 16 + lgrp * 4 + r;
                float v = acc[0][i][j][r];
                if constexpr (GATE_UP) v = silu(v) * acc[NW - 1][i][j][r];
                if (m < M && n < N) y[static_cast<size_t>(m) * N + n] = to_out<OutT>(v);
            }
        }
    }
}

template <int BM, int BN, bool GATE_UP, int PF>
hipError_t launch_mfma(const Problem& p) {
    const uint32_t m_tiles = (p.M + BM - 1) / BM;
    const uint32_t n_tiles = (p.N + BN - 1) / BN;
    const uint64_t total64 = static_cast<uint64_t>(m_tiles) * n_tiles;
    if (total64 > 0x7fffffffull) return hipErrorInvalidConfiguration;
    const uint32_t total = static_cast<uint32_t>(total64);
    const uint32_t per_xcd = (total + 7u) / 8u;
    const dim3 grid(per_xcd * 8u), block(256);
    const auto* x = static_cast<const uint16_t*>(p.x);
    const auto* wg = static_cast<const uint8_t*>(p.w);
    const auto* wu = static_cast<const uint8_t*>(p.w_up);
    if (p.out == OutType::F32) {
        hipLaunchKernelGGL((mfma_kernel<BM, BN, GATE_UP, PF, float>), grid, block, 0, p.stream, x, wg, wu,
                           static_cast<float*>(p.y), p.M, p.N, p.K, m_tiles, total, per_xcd);
    } else {
        hipLaunchKernelGGL((mfma_kernel<BM, BN, GATE_UP, PF, _Float16>), grid, block, 0, p.stream, x, wg,
                           wu, static_cast<_Float16*>(p.y), p.M, p.N, p.K, m_tiles, total, per_xcd);
    }
    return hipGetLastError();
}

#define MOTE_MFMA(BM, BN, PF)                                                                   \
    Variant{"mfma_m" #BM "_n" #BN "_p" #PF, Kind::Mfma, BM, BN, PF, &launch_mfma<BM, BN, false, PF>}, \
    Variant{"gateup_mfma_m" #BM "_n" #BN "_p" #PF, Kind::GateUpMfma, BM, BN, PF,                    \
            &launch_mfma<BM, BN, true, PF>}

const Variant kMfma[] = {
    MOTE_MFMA(64, 64, 1), MOTE_MFMA(128, 64, 1), MOTE_MFMA(64, 128, 1), MOTE_MFMA(128, 128, 1),
    MOTE_MFMA(128, 64, 3), MOTE_MFMA(128, 128, 2),
};

#undef MOTE_MFMA

}  // namespace

const Variant* mfma_variants(int* count) {
    *count = static_cast<int>(sizeof(kMfma) / sizeof(kMfma[0]));
    return kMfma;
}

bool mfma_supports(const Variant& v, const Problem& p) {
    (void)v;
    const bool up_ok = p.w_up == nullptr || reinterpret_cast<uintptr_t>(p.w_up) % 4 == 0;
    return p.K % 64 == 0 && p.K > 0 && up_ok &&
           reinterpret_cast<uintptr_t>(p.w) % 4 == 0 &&
           reinterpret_cast<uintptr_t>(p.x) % 16 == 0;
}

}  // namespace mote::q4_0

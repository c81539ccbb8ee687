// Q4_0 prefill-shaped linear (M >= 64) on the CDNA4 matrix cores with the
// weights staged in LDS as raw Q4_0 bytes, plus the fused gate/up variant.
//
//   y[m, n] = sum_k x[m, k] * w[n, k]                                (linear)
//   y[m, n] = silu(sum_k x w_gate[n, k]) * (sum_k x w_up[n, k])       (gate/up)
//
// The linear is the operation of crates/mote-backend-hip/src/
// quantized_linear.hip:13-52 (oracle crates/mote-reference/src/quantized.rs:
// 89-144); the fused gate/up has no counterpart in the reference.
//
// One 256-thread workgroup computes a BM x BN output tile with WM x (4 / WM)
// waves, each wave a (BM / WM) x (BN / (4 / WM)) grid of MFMA tiles: 16 x 16
// tiles of v_mfma_f32_16x16x32_f16, or (T32) 32 x 32 tiles of
// v_mfma_f32_32x32x16_f16, which measured 2.2-2.4 PFLOP/s on MI355X against
// 0.86-1.3 PFLOP/s for the 16 x 16 form (one to four waves per SIMD).
// K advances one Q4_0 block pair (64 elements) per step through a
// double-buffered LDS stage, one barrier per step:
//  * activations: BM rows x 64 f16 copied from HBM, stored in the k order of
//    the nibble unpacking (below), rows padded to 144 bytes so the 16 rows of
//    an MFMA operand fall on distinct banks;
//  * weights: BN rows x 36 bytes, the block pair's bytes re-aligned so every
//    nibble dword is dword aligned: [d0 | d1 << 16][block 0 nibble dwords 0-3]
//    [block 1 nibble dwords 0-3].  36 bytes per row and step, against 128 for
//    dequantised f16: the LDS traffic of the weight operand drops by 3.5x and
//    each wave dequantises the operands it feeds to its own MFMAs, in registers,
//    (q - 8) * d exactly as the skinny kernel does (exact q - 8 from the
//    1024 + q and 64 + q exponent tricks, one binary16 rounding of the
//    product).
// A 32-element block is split into four k groups g = 0..3: nibble bytes
// 4g..4g+3, elements [4g, 4g+2, 4g+1, 4g+3, 16+4g, 16+4g+2, 16+4g+1,
// 16+4g+3]; a 16 x 16 x 32 MFMA spans one block, lane group g (lanes
// 16g..16g+15) taking group g of both operands; a 32 x 32 x 16 MFMA spans two
// groups, 2h and 2h + 1 in its h-th half block, lane half c (lanes 32c..32c+31)
// taking group 2h + c.  Activations and weights agree on k either way.
//
// Q8_0 weights (Q8): a pair is staged as 17 dwords, [d0 | d1 << 16][block 0
// bytes 0-31][block 1 bytes 0-31] (block 0's bytes re-aligned); k group g is
// bytes 8g..8g+7 of a block, elements [8g, 8g+2, 8g+1, 8g+3, 8g+4, 8g+6,
// 8g+5, 8g+7], dequantised by dequant8_q8 into a binary16 hi + lo pair that
// feeds two MFMAs, and the activations are staged in that order.  A single
// binary16 product rounds (q - 8) d, up to 14 significant bits, to 11 (a
// relative error of at most 2^-11 per weight); that is well inside the
// tolerance for Q4_0's 4-bit values but measured too coarse for 8-bit ones.
#include "common.hpp"
#include "q4_0.hpp"

#include <type_traits>

namespace mote::q4_0 {
namespace {

template <int BM, int BN, bool GATE_UP, typename OutT, bool Q8 = false, int WM = 2, bool T32 = false,
          bool SPEC = false, int KP = 1>
__global__ __launch_bounds__(SPEC ? 512 : 256) void prefill_kernel(const uint16_t* __restrict__ x,
                                                      const uint8_t* __restrict__ wg,
                                                      const uint8_t* __restrict__ wu,
                                                      OutT* __restrict__ y, uint32_t M, uint32_t N,
                                                      uint32_t K, uint32_t m_tiles, uint32_t total,
                                                      uint32_t per_xcd) {
    constexpr int NW = GATE_UP ? 2 : 1;
    constexpr int WN = 4 / WM;                // waves along N
    constexpr int T = T32 ? 32 : 16;          // MFMA tile edge
    constexpr int TM = BM / (WM * T);         // MFMA tiles per wave along M
    constexpr int TN = BN / (WN * T);         // along N
    // KP block pairs (64 k each) per step and barrier (KP > 1: the pipelined
    // 32 x 32 Q4_0 step with staging waves only).
    static_assert(KP == 1 || (SPEC && T32), "several pairs per step: the pipelined step");
    constexpr int kXRow = 128 * KP + 16;      // LDS bytes per activation row and step (+16: banks)
    constexpr int XC = BM * 8 * KP / 256;     // 16-byte activation chunks per thread and step
    constexpr int WI = (BN * KP + 255) / 256; // weight (row, pair) units per thread and step (per matrix)
    static_assert((WM == 1 || WM == 2 || WM == 4) && TM >= 1 && TN >= 1 && BM % (WM * T) == 0 &&
                      BN % (WN * T) == 0 && XC >= 1, "tile shape");
    using Acc = std::conditional_t<T32, f32x16, f32x4>;
    constexpr int kAccRows = T32 ? 16 : 4;    // accumulator registers per lane and tile
    static_assert(!(Q8 && GATE_UP), "the fused gate/up is a Q4_0 operation");
    constexpr int kDw = Q8 ? 17 : 9;         // dwords of a staged block pair
    // LDS bytes per weight row and step: KP staged pairs, plus a dword when
    // that keeps the row stride odd in dwords (the 32 rows of an operand on
    // distinct banks)
    constexpr int kWRow = (kDw * KP + (KP % 2 == 0 ? 1 : 0)) * 4;
    constexpr uint32_t kPB = Q8 ? kQ8PairBytes : kPairBytes;

    __shared__ __attribute__((aligned(16))) uint8_t xs[2][BM * kXRow];
    __shared__ __attribute__((aligned(16))) uint8_t ws[NW][2][BN * kWRow];

    const uint32_t logical = (blockIdx.x % 8u) * per_xcd + blockIdx.x / 8u;
    if (logical >= total) return;
    const uint32_t tile_n = logical / m_tiles;
    const uint32_t tile_m = logical - tile_n * m_tiles;
    const uint32_t m0 = tile_m * BM;
    const uint32_t n0 = tile_n * BN;

    // SPEC: waves 4-7 only stage (loads, LDS stores) and waves 0-3 only
    // multiply, so each SIMD interleaves a staging wave's memory work with a
    // compute wave's MFMAs; both meet at the one barrier per step.
    const int tid = static_cast<int>(threadIdx.x) & 255;  // staging thread / compute thread index
    const bool stager = SPEC && threadIdx.x >= 256;       // uniform over a wave
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const uint32_t npairs = K >> 6;
    const uint32_t nsteps = npairs / KP;
    const size_t row_bytes = static_cast<size_t>(npairs) * kPB;
    const uint8_t* wsrc[NW] = {wg};
    if constexpr (GATE_UP) wsrc[1] = wu;

    // Activation chunks: chunk c of the tile is 16 bytes (8 halves) of row
    // (c / 8) % BM, pair (c / 8) / BM of the step, whose chunk c % 8 holds
    // elements 8 (c % 4) .. + 7 of block (c % 8) / 4.  One store instruction
    // covers one pair of consecutive rows, whose 16-byte row padding spreads
    // them over the banks (the two pairs of a row lie 128 bytes apart, on the
    // same banks).
    const uint16_t* xptr[XC];
    int xoff[XC];
#pragma unroll
    for (int j = 0; j < XC; ++j) {
        const int c = tid + 256 * j;
        const int row = (c >> 3) % BM, pair = (c >> 3) / BM, chunk = c & 7;
        const uint32_t m = min(m0 + row, M - 1);
        xptr[j] = x + static_cast<size_t>(m) * K + pair * 64 + chunk * 8;
        const int blk = chunk >> 2, kin = (chunk & 3) * 8;
        if constexpr (Q8)  // k group chunk % 4: both halves together
            xoff[j] = row * kXRow + pair * 128 + blk * 64 + (chunk & 3) * 16;
        else
            xoff[j] = row * kXRow + pair * 128 + blk * 64 + ((kin & 15) >> 2) * 16 + (kin >= 16 ? 8 : 0);
    }
    // Weight units: thread t copies unit t, t + 256, ... of the step, unit u
    // being block pair u % KP of row u / KP: a load instruction reads KP
    // neighbouring pairs of 64 / KP rows.  (One pair of 64 consecutive rows
    // per instruction would keep the LDS stores free of bank conflicts, but
    // measured slower with 4 pairs per step: 30.2 against 27.6 us at 128 x
    // 4096 x 14 336, 110.6 against 95.3 us for the gate/up at 64 x 8192 x
    // 28 672; level with 2.)
    const uint8_t* wptr[NW][WI];
    bool wlive[WI];
    int woff[WI];
#pragma unroll
    for (int j = 0; j < WI; ++j) {
        const int u = tid + 256 * j;
        wlive[j] = u < BN * KP;
        const int row = wlive[j] ? u / KP : 0, pair = wlive[j] ? u % KP : 0;
        woff[j] = row * kWRow + pair * kDw * 4;
        const uint32_t n = min(n0 + static_cast<uint32_t>(row), N - 1);
#pragma unroll
        for (int s = 0; s < NW; ++s) wptr[s][j] = wsrc[s] + static_cast<size_t>(n) * row_bytes + pair * kPB;
    }

    u32x4 xreg[XC];
    uint32_t wreg[NW][WI][kDw];
    auto load_stage = [&](uint32_t kp) {
        kp = min(kp, nsteps - 1);  // past the end: a cached re-read, never used
#pragma unroll
        for (int j = 0; j < XC; ++j)
            xreg[j] = *reinterpret_cast<const u32x4*>(xptr[j] + static_cast<size_t>(kp) * 64 * KP);
#pragma unroll
        for (int s = 0; s < NW; ++s)
#pragma unroll
            for (int j = 0; j < WI; ++j)
                if (wlive[j]) {
                    const uint8_t* src = wptr[s][j] + static_cast<size_t>(kp) * kPB * KP;
                    if constexpr (Q8)
                        load_pair_q8(src, wreg[s][j]);
                    else
                        load_pair(src, wreg[s][j]);
                }
    };
    auto store_stage = [&](int buf) {
#pragma unroll
        for (int j = 0; j < XC; ++j) {
            const u32x4 v = xreg[j];
            u32x2 a, b;
            a.x = __builtin_amdgcn_perm(v.y, v.x, 0x05040100u);  // (x0, x2)
            a.y = __builtin_amdgcn_perm(v.y, v.x, 0x07060302u);  // (x1, x3)
            b.x = __builtin_amdgcn_perm(v.w, v.z, 0x05040100u);  // (x4, x6)
            b.y = __builtin_amdgcn_perm(v.w, v.z, 0x07060302u);  // (x5, x7)
            *reinterpret_cast<u32x2*>(&xs[buf][xoff[j]]) = a;
            *reinterpret_cast<u32x2*>(&xs[buf][xoff[j] + (Q8 ? 8 : 16)]) = b;
        }
#pragma unroll
        for (int s = 0; s < NW; ++s)
#pragma unroll
            for (int j = 0; j < WI; ++j) {
                if (!wlive[j]) continue;
                const uint32_t (&d)[kDw] = wreg[s][j];
                uint32_t* dst = reinterpret_cast<uint32_t*>(&ws[s][buf][woff[j]]);
                if constexpr (Q8) {
                    dst[0] = __builtin_amdgcn_perm(d[8], d[0], 0x07060100u);  // d0 (bytes 0-1) | d1 (bytes 34-35)
#pragma unroll
                    for (int i = 0; i < 16; ++i) dst[1 + i] = q8_bytes(d, i);
                } else {
                    dst[0] = __builtin_amdgcn_perm(d[4], d[0], 0x07060100u);  // d0 (bytes 0-1) | d1 (bytes 18-19)
                    dst[1] = __builtin_amdgcn_perm(d[1], d[0], 0x05040302u);  // block 0 nibble bytes 0-3
                    dst[2] = __builtin_amdgcn_perm(d[2], d[1], 0x05040302u);
                    dst[3] = __builtin_amdgcn_perm(d[3], d[2], 0x05040302u);
                    dst[4] = __builtin_amdgcn_perm(d[4], d[3], 0x05040302u);
                    dst[5] = d[5]; dst[6] = d[6]; dst[7] = d[7]; dst[8] = d[8];
                }
            }
    };

    Acc acc[NW][TM][TN];
#pragma unroll
    for (int s = 0; s < NW; ++s)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < kAccRows; ++r) acc[s][i][j][r] = 0.0f;

    const DequantConsts dq = dequant_consts();
    const int lrow = lane % T;  // row of the activation operand, column of the weight operand
    const int lgrp = lane / T;  // k group (16 x 16) or lane half (32 x 32)
    const int a_base = (wm * (BM / WM) + lrow) * kXRow;
    const int b_base = (wn * (BN / WN) + lrow) * kWRow;
    auto mfma = [](const f16x8& a, const f16x8& b, const Acc& c) {
        if constexpr (T32)
            return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    };

    // Scales past binary16 range go through the scaled MFMA (common.hpp).
    constexpr uint32_t kBig = Q8 ? kQ8BigScale : kQ4BigScale;
    constexpr float kDown = Q8 ? kQ8BigDown : kQ4BigDown;
    // The step of the 32 x 32 tiles with staging waves (Q4_0 and Q8_0), software
    // pipelined: its four k groups (block, half) run as read -> dequantise ->
    // MFMA stages one group apart, so the LDS reads and the vector-ALU
    // dequantisation of group g + 1 issue while the matrix core works on
    // group g (measured 2-3 % faster than the step below at 128-512 tokens).
    auto mma_step_pipe = [&](int buf) {
        // group grp: pair grp / 4 of the step, block (grp / 2) % 2 of the
        // pair, half grp % 2 of the block
        constexpr int NG = 4 * KP;
        constexpr int QW = Q8 ? 2 : 1;   // weight dwords per lane and group
        constexpr int NB = Q8 ? 2 : 1;   // binary16 operands per weight operand (Q8_0: hi + lo)
        uint32_t scales[KP][NW][TN];
        uint32_t q[2][NW][TN][QW];
        f16x8 a[2][TM];
        f16x8 b[2][NW][TN][NB];
        auto read_b = [&](int grp, uint32_t (&dst)[NW][TN][QW]) {
            const int pair = grp >> 2, blk = (grp >> 1) & 1, g = 2 * (grp & 1) + lgrp;
#pragma unroll
            for (int s = 0; s < NW; ++s)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    // Q4_0: nibble dword g of the block; Q8_0: its bytes 8g .. 8g + 7
                    const uint32_t* src = reinterpret_cast<const uint32_t*>(
                        &ws[s][buf][b_base + j * T * kWRow + pair * kDw * 4 + 4 + blk * (16 * QW) + g * (4 * QW)]);
#pragma unroll
                    for (int w = 0; w < QW; ++w) dst[s][j][w] = src[w];
                }
        };
        auto read_a = [&](int grp, f16x8 (&dst)[TM]) {
            const int pair = grp >> 2, blk = (grp >> 1) & 1, g = 2 * (grp & 1) + lgrp;
#pragma unroll
            for (int i = 0; i < TM; ++i)
                dst[i] = *reinterpret_cast<const f16x8*>(
                    &xs[buf][a_base + i * T * kXRow + pair * 128 + blk * 64 + g * 16]);
        };
        auto dequant = [&](int grp, const uint32_t (&qq)[NW][TN][QW], f16x8 (&dst)[NW][TN][NB]) {
            const int pair = grp >> 2, blk = (grp >> 1) & 1;
#pragma unroll
            for (int s = 0; s < NW; ++s)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const f16x2 d = as_h2(__builtin_amdgcn_perm(scales[pair][s][j], scales[pair][s][j],
                                                                blk ? 0x03020302u : 0x01000100u));
                    if constexpr (Q8) {
                        const F16x8Pair v = dequant8_q8(qq[s][j][0], qq[s][j][QW - 1], d, dq.q8);
                        dst[s][j][0] = v.hi;
                        dst[s][j][NB - 1] = v.lo;
                    } else {
                        dst[s][j][0] = dequant8(qq[s][j][0], d, dq.c1024, dq.c64);
                    }
                }
        };
#pragma unroll
        for (int p = 0; p < KP; ++p)
#pragma unroll
            for (int s = 0; s < NW; ++s)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    scales[p][s][j] = *reinterpret_cast<const uint32_t*>(
                        &ws[s][buf][b_base + j * T * kWRow + p * kDw * 4]);
        read_b(0, q[0]);
        read_a(0, a[0]);
        bool big = false;
#pragma unroll
        for (int p = 0; p < KP; ++p)
#pragma unroll
            for (int s = 0; s < NW; ++s)
#pragma unroll
                for (int j = 0; j < TN; ++j) big = big || big_scales<kBig>(scales[p][s][j]);
        // the scaled MFMA of a step with a scale past binary16 range, as below
        const bool big_step = wave_any(big);
        if (__builtin_expect(big_step, 0)) {
            const f16x2 dd = {static_cast<_Float16>(kDown), static_cast<_Float16>(kDown)};
#pragma unroll
            for (int p = 0; p < KP; ++p)
#pragma unroll
                for (int s = 0; s < NW; ++s)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        scales[p][s][j] = __builtin_bit_cast(uint32_t, as_h2(scales[p][s][j]) * dd);
#pragma unroll
            for (int s = 0; s < NW; ++s)
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) acc[s][i][j] *= kDown;
        }
        dequant(0, q[0], b[0]);
#pragma unroll
        for (int grp = 0; grp < NG; ++grp) {
            const int cur = grp & 1, nxt = cur ^ 1;
            if (grp + 1 < NG) {
                read_b(grp + 1, q[nxt]);
                read_a(grp + 1, a[nxt]);
            }
#pragma unroll
            for (int s = 0; s < NW; ++s)
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int h = 0; h < NB; ++h) acc[s][i][j] = mfma(a[cur][i], b[cur][s][j][h], acc[s][i][j]);
            if (grp + 1 < NG) dequant(grp + 1, q[nxt], b[nxt]);
        }
        if (__builtin_expect(big_step, 0)) {
#pragma unroll
            for (int s = 0; s < NW; ++s)
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) acc[s][i][j] *= 1.0f / kDown;
        }
    };
    auto mma_step = [&](int buf) {
        if constexpr (SPEC && T32) {
            mma_step_pipe(buf);
            return;
        }
        uint32_t scales[NW][TN];
        bool big = false;
#pragma unroll
        for (int s = 0; s < NW; ++s)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                scales[s][j] = *reinterpret_cast<const uint32_t*>(&ws[s][buf][b_base + j * T * kWRow]);
                big = big || big_scales<kBig>(scales[s][j]);
            }
        // The step's MFMAs with the scale words sc (block 0's scale in the low
        // half, block 1's in the high half of each weight row's word).
        auto body = [&](const uint32_t (&sc)[NW][TN]) {
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
            for (int h = 0; h < (T32 ? 2 : 1); ++h) {
                const int g = T32 ? 2 * h + lgrp : lgrp;  // k group of this lane's operands
                f16x8 a[TM];
#pragma unroll
                for (int i = 0; i < TM; ++i)
                    a[i] = *reinterpret_cast<const f16x8*>(&xs[buf][a_base + i * T * kXRow + blk * 64 + g * 16]);
#pragma unroll
                for (int s = 0; s < NW; ++s) {
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        const f16x2 d = as_h2(__builtin_amdgcn_perm(sc[s][j], sc[s][j],
                                                                    blk ? 0x03020302u : 0x01000100u));
                        if constexpr (Q8) {
                            // two dword reads: the 68-byte rows keep the pair only dword aligned
                            const uint32_t* q = reinterpret_cast<const uint32_t*>(
                                &ws[s][buf][b_base + j * T * kWRow + 4 + blk * 32 + g * 8]);
                            const F16x8Pair b = dequant8_q8(q[0], q[1], d, dq.q8);
#pragma unroll
                            for (int i = 0; i < TM; ++i) {
                                acc[s][i][j] = mfma(a[i], b.hi, acc[s][i][j]);
                                acc[s][i][j] = mfma(a[i], b.lo, acc[s][i][j]);
                            }
                        } else {
                            const uint32_t q = *reinterpret_cast<const uint32_t*>(
                                &ws[s][buf][b_base + j * T * kWRow + 4 + blk * 16 + g * 4]);
                            const f16x8 b = dequant8(q, d, dq.c1024, dq.c64);
#pragma unroll
                            for (int i = 0; i < TM; ++i) acc[s][i][j] = mfma(a[i], b, acc[s][i][j]);
                        }
                    }
                }
            }
        }
        };
        // A step with a scale past binary16 range runs with every scale times
        // 2^-S and the accumulators scaled by 2^-S before and by 2^S after
        // (common.hpp).
        const bool big_step = wave_any(big);
        if (__builtin_expect(big_step, 0)) {
            const f16x2 dd = {static_cast<_Float16>(kDown), static_cast<_Float16>(kDown)};
#pragma unroll
            for (int s = 0; s < NW; ++s)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    scales[s][j] = __builtin_bit_cast(uint32_t, as_h2(scales[s][j]) * dd);
#pragma unroll
                    for (int i = 0; i < TM; ++i) acc[s][i][j] *= kDown;
                }
        }
        body(scales);
        if (__builtin_expect(big_step, 0)) {
#pragma unroll
            for (int s = 0; s < NW; ++s)
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) acc[s][i][j] *= 1.0f / kDown;
        }
    };

    // Step k: write step k + 1 (loaded during step k - 1) to the other LDS
    // buffer, issue the loads of step k + 2, multiply step k, barrier.
    if (!SPEC || stager) {
        load_stage(0);
        store_stage(0);
        load_stage(1);
    }
    __syncthreads();
    if constexpr (SPEC) {
        if (stager) {
            for (uint32_t kp = 0; kp < nsteps; ++kp) {
                if (kp + 1 < nsteps) {  // uniform
                    store_stage(static_cast<int>(kp & 1u) ^ 1);
                    load_stage(kp + 2);
                }
                __syncthreads();
            }
            return;  // the compute waves hold the results
        }
        for (uint32_t kp = 0; kp < nsteps; ++kp) {
            mma_step(static_cast<int>(kp & 1u));
            __syncthreads();
        }
    } else {
        for (uint32_t kp = 0; kp < nsteps; ++kp) {
            const int buf = static_cast<int>(kp & 1u);
            if (kp + 1 < nsteps) {  // uniform
                store_stage(buf ^ 1);
                load_stage(kp + 2);
            }
            mma_step(buf);
            __syncthreads();
        }
    }

    // Epilogue: lane holds column lrow of each tile, rows 4 lgrp + r (16 x 16)
    // or 8 (r / 4) + 4 lgrp + r % 4 (32 x 32).
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint32_t n = n0 + wn * (BN / WN) + j * T + lrow;
#pragma unroll
            for (int r = 0; r < kAccRows; ++r) {
                const int row = T32 ? 8 * (r / 4) + 4 * lgrp + r % 4 : 4 * lgrp + r;
                const uint32_t m = m0 + wm * (BM / WM) + i * T + row;
                float v = acc[0][i][j][r];
                if constexpr (GATE_UP) v = silu(v) * acc[NW - 1][i][j][r];
                if (m < M && n < N) y[static_cast<size_t>(m) * N + n] = to_out<OutT>(v);
            }
        }
    }
}

template <int BM, int BN, bool GATE_UP, bool Q8 = false, int WM = 2, bool T32 = false, bool SPEC = false,
          int KP = 1>
hipError_t launch_prefill(const Problem& p) {
    if (p.K % (64u * KP) != 0) return hipErrorInvalidValue;
    const uint32_t m_tiles = (p.M + BM - 1) / BM;
    const uint32_t n_tiles = (p.N + BN - 1) / BN;
    const uint64_t total64 = static_cast<uint64_t>(m_tiles) * n_tiles;
    if (total64 > 0x7fffffffull) return hipErrorInvalidConfiguration;
    const uint32_t total = static_cast<uint32_t>(total64);
    const uint32_t per_xcd = (total + 7u) / 8u;
    const dim3 grid(per_xcd * 8u), block(SPEC ? 512 : 256);
    const auto* x = static_cast<const uint16_t*>(p.x);
    const auto* wg = static_cast<const uint8_t*>(p.w);
    const auto* wu = static_cast<const uint8_t*>(p.w_up);
    if (p.out == OutType::F32) {
        hipLaunchKernelGGL((prefill_kernel<BM, BN, GATE_UP, float, Q8, WM, T32, SPEC, KP>), grid, block, 0, p.stream, x, wg, wu,
                           static_cast<float*>(p.y), p.M, p.N, p.K, m_tiles, total, per_xcd);
    } else {
        hipLaunchKernelGGL((prefill_kernel<BM, BN, GATE_UP, _Float16, Q8, WM, T32, SPEC, KP>), grid, block, 0, p.stream, x, wg,
                           wu, static_cast<_Float16*>(p.y), p.M, p.N, p.K, m_tiles, total, per_xcd);
    }
    return hipGetLastError();
}

#define MOTE_PREFILL(BM, BN)                                                                      \
    Variant{"mfma_r_m" #BM "_n" #BN, Kind::Mfma, BM, BN, 1, &launch_prefill<BM, BN, false>}
#define MOTE_PREFILL_GU(BM, BN)                                                                   \
    Variant{"gateup_mfma_r_m" #BM "_n" #BN, Kind::GateUpMfma, BM, BN, 1, &launch_prefill<BM, BN, true>}
#define MOTE_PREFILL_Q8(BM, BN)                                                                   \
    Variant{"q8_mfma_r_m" #BM "_n" #BN, Kind::Q8Prefill, BM, BN, 1, &launch_prefill<BM, BN, false, true>}
// 32 x 32 x 16 MFMA tiles, WM waves along M.
#define MOTE_PREFILL_X32(BM, BN, WM)                                                                 \
    Variant{"mfma_x32_m" #BM "_n" #BN "_w" #WM, Kind::Mfma, BM, BN, 1,                               \
            &launch_prefill<BM, BN, false, false, WM, true>}
#define MOTE_PREFILL_X32S(BM, BN, WM)                                                                \
    Variant{"mfma_x32s_m" #BM "_n" #BN "_w" #WM, Kind::Mfma, BM, BN, 1,                              \
            &launch_prefill<BM, BN, false, false, WM, true, true>}
// ... with KP block pairs per step (p2 = KP: K a multiple of 64 KP).
#define MOTE_PREFILL_X32SK(BM, BN, WM, KP)                                                           \
    Variant{"mfma_x32s_m" #BM "_n" #BN "_w" #WM "_k" #KP, Kind::Mfma, BM, BN, KP,                    \
            &launch_prefill<BM, BN, false, false, WM, true, true, KP>}
#define MOTE_PREFILL_GU_X32SK(BM, BN, WM, KP)                                                        \
    Variant{"gateup_mfma_x32s_m" #BM "_n" #BN "_w" #WM "_k" #KP, Kind::GateUpMfma, BM, BN, KP,       \
            &launch_prefill<BM, BN, true, false, WM, true, true, KP>}
#define MOTE_PREFILL_Q8_X32SK(BM, BN, WM, KP)                                                        \
    Variant{"q8_mfma_x32s_m" #BM "_n" #BN "_w" #WM "_k" #KP, Kind::Q8Prefill, BM, BN, KP,            \
            &launch_prefill<BM, BN, false, true, WM, true, true, KP>}
#define MOTE_PREFILL_GU_X32S(BM, BN, WM)                                                             \
    Variant{"gateup_mfma_x32s_m" #BM "_n" #BN "_w" #WM, Kind::GateUpMfma, BM, BN, 1,                 \
            &launch_prefill<BM, BN, true, false, WM, true, true>}
#define MOTE_PREFILL_Q8_X32S(BM, BN, WM)                                                             \
    Variant{"q8_mfma_x32s_m" #BM "_n" #BN "_w" #WM, Kind::Q8Prefill, BM, BN, 1,                      \
            &launch_prefill<BM, BN, false, true, WM, true, true>}

// The tiles the dispatch heuristic picks (32 x 32 MFMA tiles with staging
// waves where about one tile per CU fits, 16 x 16 tiles below that) and the
// measured alternatives of the same tile without staging waves and with
// 16 x 16 MFMAs.
const Variant kPrefill[] = {
    MOTE_PREFILL(128, 128), MOTE_PREFILL(64, 128), MOTE_PREFILL(64, 64),
    MOTE_PREFILL_GU(128, 64), MOTE_PREFILL_GU(64, 64),
    MOTE_PREFILL_Q8(64, 64),
    MOTE_PREFILL_X32(128, 128, 1),
    MOTE_PREFILL_X32S(128, 128, 1), MOTE_PREFILL_X32S(64, 128, 1), MOTE_PREFILL_X32S(128, 256, 1),
    MOTE_PREFILL_X32SK(128, 128, 1, 2), MOTE_PREFILL_X32SK(64, 128, 1, 2), MOTE_PREFILL_X32SK(128, 256, 1, 2),
    MOTE_PREFILL_X32SK(64, 128, 1, 4), MOTE_PREFILL_X32SK(64, 64, 2, 4), MOTE_PREFILL_X32SK(64, 64, 2, 2),
    MOTE_PREFILL_GU_X32SK(128, 128, 1, 2), MOTE_PREFILL_GU_X32SK(64, 128, 1, 2),
    MOTE_PREFILL_GU_X32SK(64, 128, 1, 4), MOTE_PREFILL_GU_X32SK(64, 64, 2, 4),
    MOTE_PREFILL_GU_X32S(128, 128, 1), MOTE_PREFILL_GU_X32S(64, 128, 1),
    MOTE_PREFILL_Q8_X32S(128, 128, 1), MOTE_PREFILL_Q8_X32S(128, 256, 1),
    MOTE_PREFILL_Q8_X32SK(128, 128, 1, 2), MOTE_PREFILL_Q8_X32SK(128, 256, 1, 2),
    MOTE_PREFILL_Q8_X32SK(64, 128, 1, 2), MOTE_PREFILL_Q8_X32SK(64, 128, 1, 4),
};

#undef MOTE_PREFILL
#undef MOTE_PREFILL_GU
#undef MOTE_PREFILL_Q8
#undef MOTE_PREFILL_X32
#undef MOTE_PREFILL_X32S
#undef MOTE_PREFILL_GU_X32S
#undef MOTE_PREFILL_X32SK
#undef MOTE_PREFILL_Q8_X32SK
#undef MOTE_PREFILL_GU_X32SK
#undef MOTE_PREFILL_Q8_X32S

}  // namespace

const Variant* prefill_variants(int* count) {
    *count = static_cast<int>(sizeof(kPrefill) / sizeof(kPrefill[0]));
    return kPrefill;
}

// K a multiple of 64, x 16-byte and the weights (and the up matrix of a
// gate/up) dword aligned; any M and N (partial tiles are masked).
bool prefill_supports(const Variant& v, const Problem& p) {
    const bool up_ok = p.w_up == nullptr || reinterpret_cast<uintptr_t>(p.w_up) % 4 == 0;
    const uint32_t step = 64u * static_cast<uint32_t>(v.p2 > 0 ? v.p2 : 1);
    return p.K % step == 0 && p.K > 0 && up_ok && reinterpret_cast<uintptr_t>(p.w) % 4 == 0 &&
           reinterpret_cast<uintptr_t>(p.x) % 16 == 0;
}

}  // namespace mote::q4_0

// The Q4_0 / Q8_0 skinny-GEMM kernel (q4_0_skinny_mfma.hip describes the
// mapping and launches it), templated on a timeline policy, so that the probe
// library can instantiate the very kernel the library ships with per-wave
// timestamps (mote_amd/probes/skinny_probe.hip) while the library
// instantiates the policy that does nothing (NoSkinnyTimeline: every hook is
// empty, and the code is that of the kernel without hooks); and the grid the
// launcher computes for it (skinny_grid).
#pragma once

#include "common.hpp"
#include "q4_0.hpp"

#include <type_traits>

namespace mote::q4_0 {
namespace {

// Timeline hooks of skinny_mfma_kernel (the deferred-reduction path): begin
// (wave start), x_ready (the wave's activations converted to MFMA operands),
// landed / issued (item i's weights in the wave's stage / its MFMAs issued),
// reduced (the partial tiles summed and stored), end (the wave's last
// instruction).
struct NoSkinnyTimeline {
    __device__ explicit NoSkinnyTimeline(uint32_t*) {}
    __device__ __forceinline__ void begin() {}
    __device__ __forceinline__ void x_ready() {}
    __device__ __forceinline__ void landed(int) {}
    __device__ __forceinline__ void issued(int) {}
    __device__ __forceinline__ void reduced() {}
    __device__ __forceinline__ void end() {}
};

__device__ __forceinline__ uint32_t pick(const uint32_t* x, int a, int b) {
    const uint32_t lo = (a & 1) ? 0x0302u : 0x0100u;
    const uint32_t hi = (b & 1) ? 0x07060000u : 0x05040000u;
    return __builtin_amdgcn_perm(x[b >> 1], x[a >> 1], hi | lo);
}

// Split-K epilogue: y[i] = sum over the K parts of part[k][i], in part order
// (deterministic), converted to the output type; gate/up (GU): silu of the
// gate sum times the up sum, the up planes following the kparts gate planes.
// Up to kMaxParts parts every load of an element is issued before the first
// add (one memory latency instead of one per part); more parts loop.
constexpr uint32_t kMaxParts = 16;

// SYS: the loads are system-scope (they miss in every cache and read what the
// write-through partial stores of other workgroups left in memory).
template <bool SYS = false>
__device__ __forceinline__ float load_part(const float* p, uint64_t i) {
    if constexpr (SYS) return __hip_atomic_load(p + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    return p[i];
}

template <bool SYS = false>
__device__ __forceinline__ float sum_parts(const float* __restrict__ p, uint32_t kparts, uint64_t count, uint64_t i) {
    if (kparts > kMaxParts) {
        float s = load_part<SYS>(p, i);
        for (uint32_t k = 1; k < kparts; ++k) s += load_part<SYS>(p, static_cast<uint64_t>(k) * count + i);
        return s;
    }
    float v[kMaxParts];
#pragma unroll
    for (uint32_t k = 0; k < kMaxParts; ++k) v[k] = k < kparts ? load_part<SYS>(p, static_cast<uint64_t>(k) * count + i) : 0.0f;
    float s = v[0];
#pragma unroll
    for (uint32_t k = 1; k < kMaxParts; ++k)
        if (k < kparts) s += v[k];
    return s;
}

// TL: the timeline policy, constructed from `tile_count` (which the kernel
// itself reads only with split K; the probe's instantiation has no split K
// and passes its stamp buffer there).
template <int KS, int STEPS, int MT, int D, int RT, bool TR, typename OutT, int LAZY = 0, bool XC = false,
          bool GU = false, bool Q8 = false, bool XW = false, bool SK = false, class TL = NoSkinnyTimeline>
__global__ __launch_bounds__(KS * 64) void skinny_mfma_kernel(const uint16_t* __restrict__ x,
                                                             const uint8_t* __restrict__ w,
                                                             const uint8_t* __restrict__ w_up,
                                                             OutT* __restrict__ y, uint32_t M,
                                                             uint32_t N, uint32_t K,
                                                             uint32_t token_groups, uint32_t items,
                                                             uint32_t groups_per_xcd, float* __restrict__ kpartial,
                                                             uint32_t kparts, uint32_t* __restrict__ tile_count) {
    static_assert(!SK || std::is_same_v<TL, NoSkinnyTimeline>, "split K reads tile_count itself");
    TL tl(tile_count);
    // Transposed loads: wave-private staging of the raw pairs, [row tile][row]
    // [pair of the slice], rows padded by one dword so the 16 rows read by an
    // MFMA operand fall on distinct banks.
    constexpr uint32_t kPB = Q8 ? kQ8PairBytes : kPairBytes;  // bytes of a block pair
    constexpr int kDw = Q8 ? 17 : 9;                          // its dwords
    constexpr int kSlicePairs = STEPS * 4;
    constexpr int kStageRow = kSlicePairs * kPB + 4;
    constexpr int kStageBytes = TR ? KS * RT * 16 * kStageRow : 4;
    __shared__ __attribute__((aligned(16))) uint8_t stage[kStageBytes];
    // LAZY > 0: a workgroup owns at most LAZY items and its waves reduce them
    // at the end, kChunk items per barrier (as many as fit the 160 KiB of LDS
    // beside the stage, rounded down to a power of two), instead of once per
    // item.
    // XC: the activations are loaded whole cache lines per instruction (lane
    // l reads bytes 16 l .. 16 l + 15 of a 1 KiB run of the wave's slices of
    // the 16 tokens) and redistributed to the operand layout through a
    // wave-private LDS region, kXTok tokens per round.  Loaded directly, each
    // lane reads its own 128-byte pair, so every instruction touches 64 lines
    // and 16 tokens' slices outgrow the vector L1, which then refetches them.
    constexpr int kSliceBytes = STEPS * 512;  // one token's slice of x
    constexpr int kXRow = kSliceBytes + 16;
    constexpr int kXTok = 4;
    constexpr int kXBytes = XC ? KS * kXTok * kXRow : 16;
    __shared__ __attribute__((aligned(16))) uint8_t xstage[kXBytes];
    constexpr int kPartItem = KS * RT * MT * 16 * 17 * 4;
    constexpr int kFit = (160 * 1024 - kStageBytes - kXBytes) / kPartItem;
    constexpr int kChunk = LAZY == 0 ? 1 : (kFit >= LAZY ? LAZY : kFit >= 4 ? 4 : kFit >= 2 ? 2 : 1);
    static_assert(LAZY == 0 || LAZY % kChunk == 0, "chunks must tile the items");
    constexpr int kParts = kChunk * RT * MT;
    __shared__ float part[KS][kParts][16][17];

    const int tid = static_cast<int>(threadIdx.x);
    const int kw = tid >> 6;
    const int lane = tid & 63;
    const int li = lane & 15;  // row of the A operand, token of the B operand
    const int lg = lane >> 4;  // lane group: which of the step's 4 pairs
    const uint32_t npairs = K >> 6;
    const size_t row_bytes = static_cast<size_t>(npairs) * kPB;
    const uint32_t groups = gridDim.x;
    // XCD-aware order: workgroups of one XCD take consecutive items, so the
    // token tiles of a row tile read its weights through the same L2.
    const uint32_t first = (blockIdx.x % 8u) * groups_per_xcd + blockIdx.x / 8u;
    tl.begin();

    // Item -> (row tile, token group of MT 16-token tiles, K part).  The grid
    // size is a multiple of token_groups x kparts, so a workgroup keeps one
    // token group and one K part.  Split K (SK): K is cut into kparts parts of
    // KS x STEPS x 256; each item writes its part's partial sums to
    // `kpartial` ([kparts][M][N] f32; gate/up: the gate planes, then the up
    // planes), which are added in part order either by the last workgroup of
    // the tile to finish (tile_count non-null: one arrival counter per
    // (row tile, token group), zero on entry and left zero) or by a second
    // kernel.
    static_assert(!GU || RT == 2, "gate/up items are one gate and one up row tile");
    constexpr uint32_t kItemRows = GU ? 16u : 16u * RT;
    const uint32_t combos = token_groups * kparts;
    auto rows_of = [&](uint32_t item) { return (item / combos) * kItemRows; };
    const uint32_t combo = first % combos;
    const uint32_t tok0 = (combo % token_groups) * (16u * MT);
    const uint32_t kpart = combo / token_groups;
    const uint32_t pair0 = kpart * (npairs / kparts);  // first block pair of this K part

    // Weight loads of one item: RT row tiles x STEPS pairs per lane.  Direct
    // mapping: lane (li, lg) loads the pair it feeds to the MFMAs, so one
    // instruction spans 16 rows.  Transposed mapping (TR): lane l loads pair
    // l % (4 STEPS) of the wave's slice in row s (16 / STEPS) + l / (4 STEPS),
    // so one instruction spans 16 / STEPS rows of 4 STEPS neighbouring pairs,
    // and the pairs reach their MFMA lanes through the wave's LDS stage.
    constexpr int kRowsPerLoad = 16 / STEPS;
    auto load_item = [&](uint32_t item, uint32_t (&raw)[RT * STEPS][kDw]) {
        const uint32_t it = min(item, items - 1);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
            for (int s = 0; s < STEPS; ++s) {
                uint32_t r, p;
                if constexpr (TR) {
                    r = static_cast<uint32_t>(s * kRowsPerLoad + lane / kSlicePairs);
                    p = pair0 + static_cast<uint32_t>(kw * kSlicePairs + lane % kSlicePairs);
                } else {
                    r = static_cast<uint32_t>(li);
                    p = pair0 + (static_cast<uint32_t>(kw) * STEPS + s) * 4u + static_cast<uint32_t>(lg);
                }
                const uint32_t n = min(rows_of(it) + (GU ? 0u : 16u * rt) + r, N - 1);
                const uint8_t* base = (GU && rt == 1) ? w_up : w;
                const uint8_t* src = base + static_cast<size_t>(n) * row_bytes + static_cast<size_t>(p) * kPB;
                if constexpr (Q8)
                    load_pair_q8(src, raw[rt * STEPS + s]);
                else
                    load_pair(src, raw[rt * STEPS + s]);
            }
        }
    };
    uint8_t* my_stage = stage + (TR ? kw * RT * 16 * kStageRow : 0);
    auto stage_item = [&](const uint32_t (&raw)[RT * STEPS][kDw]) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int s = 0; s < STEPS; ++s) {
                const int r = s * kRowsPerLoad + lane / kSlicePairs;
                uint32_t* dst = reinterpret_cast<uint32_t*>(my_stage + (rt * 16 + r) * kStageRow +
                                                            (lane % kSlicePairs) * kPB);
#pragma unroll
                for (int i = 0; i < kDw; ++i) dst[i] = raw[rt * STEPS + s][i];
            }
    };
    auto staged_pair = [&](int rt, int s, uint32_t (&c)[kDw]) {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(my_stage + (rt * 16 + li) * kStageRow +
                                                                (4 * s + lg) * kPB);
#pragma unroll
        for (int i = 0; i < kDw; ++i) c[i] = src[i];
    };

    // The first item's weights, the activations (reused by every item), and
    // with D = 2 the second item's weights, issued before the activations are
    // waited for.
    uint32_t buf0[RT * STEPS][kDw];
    uint32_t buf1[RT * STEPS][kDw];
    // XW: the activations first, converted before any weight load is issued
    // (every CU needs all of x; with weight loads queued ahead of it, its
    // broadcast took twice as long).
    static_assert(!XW || LAZY > 0, "x first is a variant of the deferred reduction");
    static_assert(!SK || LAZY > 0, "split K adds its parts in the deferred reduction's epilogue");
    if constexpr (!XW) load_item(first, buf0);
    // Activations of this wave's K slice for the workgroup's MT token tiles.
    // Tokens past M read row M - 1: a token only feeds its own output column
    // of the MFMA, and those columns are never stored.
    constexpr int kXLoads = XC ? 16 * kSliceBytes / 1024 : 1;
    u32x4 xg[MT][kXLoads];
    u32x4 xraw[MT][STEPS][8];
    if constexpr (XC) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int c = 0; c < kXLoads; ++c) {
                const uint32_t f = static_cast<uint32_t>(c) * 1024u + static_cast<uint32_t>(lane) * 16u;
                // A load whose tokens all lie past M is not issued (uniform
                // over the workgroup): its chunks feed only columns that are
                // never stored.  Issued, every wave loaded all 16 tokens of x
                // whatever M was (measured on MI355X: 4 / 8 x 4096 x 4096 5.81
                // / 6.02 -> 5.44 / 5.52 us, 8 x 4096 x 6144 7.09 -> 6.55 us).
                if (tok0 + 16u * mt + static_cast<uint32_t>(c) * 1024u / kSliceBytes >= M) {
                    xg[mt][c] = u32x4{0u, 0u, 0u, 0u};
                    continue;
                }
                const uint32_t m = min(tok0 + 16u * mt + f / kSliceBytes, M - 1);
                const uint16_t* src = x + static_cast<size_t>(m) * K + static_cast<size_t>(pair0) * 64 +
                                      static_cast<size_t>(kw) * STEPS * 256 + (f % kSliceBytes) / 2;
                xg[mt][c] = *reinterpret_cast<const u32x4*>(src);
            }
    } else {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            // lanes of tokens past M load nothing: their columns are never stored
            const bool live = tok0 + 16u * mt + static_cast<uint32_t>(li) < M;
            const uint32_t m = min(tok0 + 16u * mt + static_cast<uint32_t>(li), M - 1);
            const uint16_t* xrow = x + static_cast<size_t>(m) * K;
#pragma unroll
            for (int s = 0; s < STEPS; ++s) {
                const uint32_t p = pair0 + (static_cast<uint32_t>(kw) * STEPS + s) * 4u + static_cast<uint32_t>(lg);
                const u32x4* src = reinterpret_cast<const u32x4*>(xrow + static_cast<size_t>(p) * 64);
                if (live) {
#pragma unroll
                    for (int c = 0; c < 8; ++c) xraw[mt][s][c] = src[c];
                } else {
#pragma unroll
                    for (int c = 0; c < 8; ++c) xraw[mt][s][c] = u32x4{0u, 0u, 0u, 0u};
                }
            }
        }
    }
    if constexpr (D == 2) load_item(first + groups, buf1);
    // Permutes the activations into the order of the weight operands (waits
    // for x; the LAZY path first stages its first item and issues the next
    // item's loads, so HBM is not idle while x is broadcast to every CU).
    f16x8 xb[MT][STEPS][8];
    auto convert_x = [&]() {
    if constexpr (XC) {
        // Round r: every lane writes the chunks of tokens r kXTok .. r kXTok +
        // kXTok - 1 it loaded, then the lanes of those tokens read their pairs
        // back (a wave's LDS operations complete in order).  Tokens past M
        // are not read back: their operands stay zero.
        uint8_t* xs = xstage + kw * kXTok * kXRow;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int s = 0; s < STEPS; ++s)
#pragma unroll
                for (int c = 0; c < 8; ++c) xraw[mt][s][c] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int r = 0; r < 16 / kXTok; ++r) {
                // Rounds of tokens past M only feed unstored columns (their
                // operands stay zero); uniform over the workgroup.
                if (tok0 + 16u * mt + static_cast<uint32_t>(r * kXTok) >= M) break;
#pragma unroll
                for (int c = 0; c < kXLoads; ++c) {
                    if ((c * 1024 / kSliceBytes) / kXTok != r) continue;  // folds after unrolling
                    const uint32_t f = static_cast<uint32_t>(c) * 1024u + static_cast<uint32_t>(lane) * 16u;
                    const uint32_t tok = f / kSliceBytes - static_cast<uint32_t>(r * kXTok);
                    *reinterpret_cast<u32x4*>(xs + tok * kXRow + f % kSliceBytes) = xg[mt][c];
                }
                if (li / kXTok == r) {
                    const uint8_t* row = xs + (li - r * kXTok) * kXRow;
#pragma unroll
                    for (int s = 0; s < STEPS; ++s)
#pragma unroll
                        for (int c = 0; c < 8; ++c)
                            xraw[mt][s][c] = *reinterpret_cast<const u32x4*>(row + (4 * s + lg) * 128 + 16 * c);
                }
            }
        }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int s = 0; s < STEPS; ++s) {
            uint32_t xr[32];
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const u32x4 v = xraw[mt][s][c];
                xr[4 * c + 0] = v.x; xr[4 * c + 1] = v.y; xr[4 * c + 2] = v.z; xr[4 * c + 3] = v.w;
            }
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                if constexpr (Q8) {  // elements 8t + [0, 2, 1, 3, 4, 6, 5, 7]
                    const int e = 8 * t;
                    const f16x2 a = as_h2(pick(xr, e, e + 2)), b = as_h2(pick(xr, e + 1, e + 3));
                    const f16x2 c = as_h2(pick(xr, e + 4, e + 6)), d = as_h2(pick(xr, e + 5, e + 7));
                    xb[mt][s][t] = f16x8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
                } else {
                    const int base = t < 4 ? 0 : 32;
                    const int e0 = base + pair_byte_element(t, 0), e1 = base + pair_byte_element(t, 1);
                    const int e2 = base + pair_byte_element(t, 2), e3 = base + pair_byte_element(t, 3);
                    const f16x2 a = as_h2(pick(xr, e0, e2)), b = as_h2(pick(xr, e1, e3));
                    const f16x2 c = as_h2(pick(xr, e0 + 16, e2 + 16)), d = as_h2(pick(xr, e1 + 16, e3 + 16));
                    xb[mt][s][t] = f16x8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
                }
            }
        }
    }
    };
    if constexpr (LAZY == 0) convert_x();
    if constexpr (XW) {
        convert_x();
        tl.x_ready();
        load_item(first, buf0);
    }
    const DequantConsts dq = dequant_consts();

    // Dequantise + MFMA one item (staged in LDS with TR, else from `buf`)
    // into `acc`.
    // Scales past binary16 range go through the scaled MFMA (common.hpp).
    constexpr uint32_t kBig = Q8 ? kQ8BigScale : kQ4BigScale;
    constexpr float kDown = Q8 ? kQ8BigDown : kQ4BigDown;
    auto mma_item = [&](const uint32_t (&buf)[RT * STEPS][kDw], f32x4 (&acc)[RT][MT]) {
#pragma unroll
        for (int s = 0; s < STEPS; ++s) {
            uint32_t q[RT][Q8 ? 16 : 8];
            f16x2 d0[RT], d1[RT];
            bool big = false;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                uint32_t c[kDw];
                if constexpr (TR) {
                    staged_pair(rt, s, c);
                } else {
#pragma unroll
                    for (int i = 0; i < kDw; ++i) c[i] = buf[rt * STEPS + s][i];
                }
                if constexpr (Q8) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) q[rt][i] = q8_bytes(c, i);
                    d1[rt] = as_h2(__builtin_amdgcn_perm(c[8], c[8], 0x03020302u));
                    big = big || big_scales<kBig>((c[0] & 0xFFFFu) | (c[8] & 0xFFFF0000u));
                } else {
                    q[rt][0] = pair_q0(c);
                    q[rt][1] = c[1]; q[rt][2] = c[2]; q[rt][3] = c[3];
                    q[rt][4] = c[5]; q[rt][5] = c[6]; q[rt][6] = c[7]; q[rt][7] = c[8];
                    d1[rt] = as_h2(__builtin_amdgcn_perm(c[4], c[4], 0x03020302u));
                    big = big || big_scales<kBig>((c[0] & 0xFFFFu) | (c[4] & 0xFFFF0000u));
                }
                d0[rt] = as_h2(__builtin_amdgcn_perm(c[0], c[0], 0x01000100u));
            }
            // The step's MFMAs with block scales e0 (dwords 0-3) and e1 (4-7).
            auto t_loop = [&](const f16x2 (&e0)[RT], const f16x2 (&e1)[RT]) {
#pragma unroll
            for (int t = 0; t < 8; ++t) {
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    if constexpr (Q8) {  // the weight as hi + lo: two MFMAs against the same x
                        const F16x8Pair a = dequant8_q8(q[rt][2 * t], q[rt][2 * t + 1], t < 4 ? e0[rt] : e1[rt], dq.q8);
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) {
                            acc[rt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.hi, xb[mt][s][t], acc[rt][mt], 0, 0, 0);
                            acc[rt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.lo, xb[mt][s][t], acc[rt][mt], 0, 0, 0);
                        }
                    } else {
                        const f16x8 a = dequant8(q[rt][t], t < 4 ? e0[rt] : e1[rt], dq.c1024, dq.c64);
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt)
                            acc[rt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, xb[mt][s][t], acc[rt][mt], 0, 0, 0);
                    }
                }
            }
            };
            // A step with a scale past binary16 range runs with every scale
            // times 2^-S and the accumulators scaled by 2^-S before and by 2^S
            // after (common.hpp).
            const bool big_step = wave_any(big);
            if (__builtin_expect(big_step, 0)) {
                const f16x2 dd = {static_cast<_Float16>(kDown), static_cast<_Float16>(kDown)};
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    d0[rt] = d0[rt] * dd;
                    d1[rt] = d1[rt] * dd;
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[rt][mt] *= kDown;
                }
            }
            t_loop(d0, d1);
            if (__builtin_expect(big_step, 0)) {
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[rt][mt] *= 1.0f / kDown;
            }
        }
    };

    // The KS partial tiles of part slot `tile` summed in slice order at
    // (row, token).
    auto tile_sum = [&](int tile, int row, int tok) {
        float sum = part[0][tile][row][tok];
#pragma unroll
        for (int k = 1; k < KS; ++k) sum += part[k][tile][row][tok];
        return sum;
    };
    // Output (m, n) from part slot `tile`; with GU, silu(gate) * up from the
    // slot's gate tile and the up tile MT slots after it (split K: both sums
    // to their planes, the second kernel applies silu(gate) * up).
    auto store = [&](uint32_t m, uint32_t n, int tile, int row, int tok) {
        if constexpr (SK) {
            float* dst = kpartial + (static_cast<size_t>(kpart) * M + m) * N + n;
            const float g = tile_sum(tile, row, tok);
            const float u = GU ? tile_sum(tile + MT, row, tok) : 0.0f;
            float* dst_u = dst + static_cast<size_t>(kparts) * M * N;
            if (tile_count != nullptr) {
                // folded epilogue: system-scope stores write through every
                // cache, so the workgroup that adds the parts can read them
                // from memory without a cache writeback
                __hip_atomic_store(dst, g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                if constexpr (GU) __hip_atomic_store(dst_u, u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            } else {
                dst[0] = g;
                if constexpr (GU) dst_u[0] = u;
            }
        } else {
            float v = tile_sum(tile, row, tok);
            if constexpr (GU) v = silu(v) * tile_sum(tile + MT, row, tok);
            y[static_cast<size_t>(m) * N + n] = to_out<OutT>(v);
        }
    };

    auto process = [&](uint32_t it, uint32_t (&buf)[RT * STEPS][kDw], uint32_t next, auto refill) {
        if constexpr (TR) {
            // LDS operations of a wave complete in order: the stage is read
            // back below, and rewritten by the next item only after this
            // item's reads.
            stage_item(buf);
            if constexpr (decltype(refill)::value) load_item(next, buf);
        }
        f32x4 acc[RT][MT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[rt][mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        mma_item(buf, acc);
        if constexpr (!TR && decltype(refill)::value) load_item(next, buf);

        // lane holds rows 4 lg + r, token li of each (row tile, token tile)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) part[kw][rt * MT + mt][4 * lg + r][li] = acc[rt][mt][r];
        __syncthreads();
        for (int o = tid; o < 256 * (GU ? 1 : RT) * MT; o += KS * 64) {
            const int row = o & 15, tok = (o >> 4) & 15, tile = o >> 8;
            const int rt = GU ? 0 : tile / MT, mt = tile % MT;
            const uint32_t n = rows_of(it) + 16u * rt + static_cast<uint32_t>(row);
            const uint32_t m = tok0 + 16u * mt + static_cast<uint32_t>(tok);
            if (n < N && m < M) store(m, n, tile, row, tok);
        }
        __syncthreads();
    };

    uint32_t item = first;
    if constexpr (LAZY > 0) {
        // Each wave streams its slice of every item of the workgroup with the
        // next item's loads in flight, independently of the other waves; the
        // partial tiles stay in registers until all items are done, then meet
        // in LDS in chunks of kChunk items.  (A second item in flight measured
        // slower: a deeper request front lowers the achieved HBM rate.)
        static_assert(D == 1, "the deferred reduction streams one item ahead");
        f32x4 accs[LAZY][RT][MT];
#pragma unroll
        for (int i = 0; i < LAZY; ++i)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) accs[i][rt][mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < LAZY; ++i) {
            const uint32_t it = first + static_cast<uint32_t>(i) * groups;
            if (it < items) {  // uniform over the workgroup
                stage_item(buf0);
                tl.landed(i);
                if (i + 1 < LAZY) load_item(it + groups, buf0);
                __builtin_amdgcn_sched_barrier(0);  // the loads go out before this item's MFMAs
                if (i == 0 && !XW) {
                    convert_x();
                    tl.x_ready();
                }
                mma_item(buf0, accs[i]);
                tl.issued(i);
            }
        }
#pragma unroll
        for (int c0 = 0; c0 < LAZY; c0 += kChunk) {
            if (c0 > 0) __syncthreads();  // the previous chunk has been read
#pragma unroll
            for (int i = 0; i < kChunk; ++i)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            part[kw][(i * RT + rt) * MT + mt][4 * lg + r][li] = accs[c0 + i][rt][mt][r];
            __syncthreads();
            for (int o = tid; o < 256 * kChunk * (GU ? 1 : RT) * MT; o += KS * 64) {
                const int row = o & 15, tok = (o >> 4) & 15, t = o >> 8;  // t: (item, [rt,] mt)
                const int i = t / ((GU ? 1 : RT) * MT), rt = GU ? 0 : (t / MT) % RT, mt = t % MT;
                const uint32_t it = first + static_cast<uint32_t>(c0 + i) * groups;
                if (it >= items) continue;
                const uint32_t n = rows_of(it) + 16u * rt + static_cast<uint32_t>(row);
                const uint32_t m = tok0 + 16u * mt + static_cast<uint32_t>(tok);
                if (n < N && m < M) store(m, n, (i * RT + rt) * MT + mt, row, tok);
            }
        }
        tl.reduced();
        if constexpr (SK) {
            if (tile_count != nullptr) {  // uniform
                // This workgroup's partial tiles are stored with system-scope
                // (write-through) stores: once every wave's stores have
                // completed (vmcnt 0, then the barrier) they are in memory,
                // and the workgroup counts itself in at each of its items'
                // tiles with a system-scope atomic.  The last of a tile's
                // kparts workgroups reads the parts with system-scope loads,
                // adds them in part order (as the second kernel would) and
                // resets the tile's counter for the next call.  (Agent-scope
                // release and acquire fences would instead write back and
                // invalidate the whole L2 of the XCD, per wave: measured over
                // six times slower than the second kernel.)
                __shared__ uint32_t last_of[LAZY];
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's partial stores are done
                __syncthreads();
                const uint32_t tok_group = combo % token_groups;
                if (tid < LAZY) {
                    const uint32_t it = first + static_cast<uint32_t>(tid) * groups;
                    uint32_t last = 0;
                    if (it < items) {
                        const uint32_t old = __hip_atomic_fetch_add(&tile_count[(it / combos) * token_groups + tok_group],
                                                                    1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                        last = old + 1u == kparts ? 1u : 0u;
                    }
                    last_of[tid] = last;
                }
                __syncthreads();
                uint32_t any = 0;
#pragma unroll
                for (int i = 0; i < LAZY; ++i) any |= last_of[i];
                if (any != 0) {  // uniform
                    const uint64_t count = static_cast<uint64_t>(M) * N;
#pragma unroll
                    for (int i = 0; i < LAZY; ++i) {
                        if (last_of[i] == 0) continue;  // uniform
                        const uint32_t it = first + static_cast<uint32_t>(i) * groups;
                        for (int o = tid; o < static_cast<int>(kItemRows) * 16 * MT; o += KS * 64) {
                            const uint32_t n = rows_of(it) + static_cast<uint32_t>(o) % kItemRows;
                            const uint32_t m = tok0 + static_cast<uint32_t>(o) / kItemRows;
                            if (n >= N || m >= M) continue;
                            const uint64_t e = static_cast<uint64_t>(m) * N + n;
                            float v = sum_parts<true>(kpartial, kparts, count, e);
                            if constexpr (GU)
                                v = silu(v) * sum_parts<true>(kpartial + static_cast<uint64_t>(kparts) * count, kparts, count, e);
                            y[e] = to_out<OutT>(v);
                        }
                        if (tid == 0)
                            __hip_atomic_store(&tile_count[(it / combos) * token_groups + tok_group], 0u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_SYSTEM);
                    }
                }
            }
        }
    } else if constexpr (TR && D == 1) {
        // The stage frees the registers as soon as an item is written to LDS,
        // so one register buffer already keeps the next item in flight.
        for (; item < items; item += groups) process(item, buf0, item + groups, std::true_type{});
    } else if constexpr (D == 1) {
        for (; item < items; item += groups) {
            // Copying the buffer waits for this item only; the next item's
            // loads then run under this item's arithmetic.
            uint32_t cur[RT * STEPS][kDw];
#pragma unroll
            for (int s = 0; s < RT * STEPS; ++s)
#pragma unroll
                for (int i = 0; i < kDw; ++i) cur[s][i] = buf0[s][i];
            load_item(item + groups, buf0);
            process(item, cur, item, std::false_type{});
        }
    } else {
        for (; item < items; item += 2 * groups) {
            process(item, buf0, item + 2 * groups, std::true_type{});
            if (item + groups < items)  // uniform
                process(item + groups, buf1, item + 3 * groups, std::true_type{});
        }
    }
    tl.end();
}

// Grid of a skinny variant: items are (row tile, token group, K part); whole
// XCD rounds (8 groups) that are also a multiple of token_groups x kparts, so
// every workgroup keeps one token group and K part (extra groups find no
// item).  ok = false: more items than a 32-bit index holds.
struct SkinnyGrid {
    uint32_t token_groups, kparts, items, groups, per_xcd;
    bool ok;
};

template <int KS, int STEPS, int MT, int G, int RT, int LAZY, bool GU, bool SK>
SkinnyGrid skinny_grid(uint32_t M, uint32_t N, uint32_t K, int cus) {
    SkinnyGrid g{};
    constexpr uint32_t kItemRows = GU ? 16u : 16u * RT;
    const uint32_t row_tiles = (N + kItemRows - 1) / kItemRows;
    g.token_groups = (M + 16 * MT - 1) / (16 * MT);
    g.kparts = SK ? K / (KS * STEPS * 256) : 1u;
    const uint64_t items64 = static_cast<uint64_t>(row_tiles) * g.token_groups * g.kparts;
    g.ok = items64 <= 0x7fffffffull;
    if (!g.ok) return g;
    g.items = static_cast<uint32_t>(items64);
    const uint32_t combos = g.token_groups * g.kparts;
    uint32_t a = 8u, b = combos;
    while (b != 0) { const uint32_t t = a % b; a = b; b = t; }
    const uint32_t unit = 8u / a * combos;  // lcm(8, combos)
    uint32_t groups = static_cast<uint32_t>(cus) * G;
    if (groups > g.items) groups = g.items;
    if (LAZY > 0 && groups < (g.items + LAZY - 1) / LAZY) groups = (g.items + LAZY - 1) / LAZY;  // <= LAZY items each
    if constexpr (LAZY > 0 && !SK && G == 1) {
        // Balanced: as few items per workgroup as one workgroup per CU allows,
        // and no more workgroups than that count needs (every workgroup loads
        // all of its token group's x, so a workgroup with fewer items than the
        // busiest adds x traffic without shortening the kernel): at 16 x 4096
        // x 14 336, 224 workgroups of 4 items took 11.3 us against 12.1 us for
        // 256 of 3 or 4; at 16 x 4096 x 6144, 192 of 2 took 7.2 against 7.9 us.
        uint32_t ipw = (g.items + cus - 1) / static_cast<uint32_t>(cus);
        if (ipw > static_cast<uint32_t>(LAZY)) ipw = LAZY;
        groups = (g.items + ipw - 1) / ipw;
    }
    g.groups = (groups + unit - 1) / unit * unit;
    g.per_xcd = g.groups / 8u;
    return g;
}

}  // namespace
}  // namespace mote::q4_0

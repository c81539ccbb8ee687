// Decode GEMV (M = 1, and 2-4 tokens) for gfx950 over GGML Q4_0 and Q8_0
// weights: persistent, software-pipelined waves.
//
// Computes y[m, n] = sum_k x[m, k] * w[n, k] for f16 x [M, K] and quantized
// w [N, K], the operation of crates/mote-backend-hip/src/
// quantized_linear.hip:13-52 (oracle crates/mote-reference/src/
// quantized.rs:89-144; Q8_0 decode at :191-195).
//
// The grid is G workgroups of 8 waves per CU.  A row group of S waves owns
// one row at a time; lane l of slice s owns block pairs s*span + l + 64 i
// (i < P, 64 elements each) of the row, so K <= 4096 P S.  Row group g walks
// rows g, g + T, g + 2T, ... (T groups in the grid), so at any moment the
// waves of the whole chip read neighbouring rows and the request front
// sweeps the matrix once, in order.  Each wave issues the loads of row j + D
// before it computes row j, so D rows are in flight behind the arithmetic
// instead of the arithmetic piling up after the last byte arrives.  D = 1
// measures fastest: a deeper front spreads the chip's outstanding requests
// over more of the matrix and lowers the achieved HBM rate, also for a pure
// read of the same pattern.
//
// Fused gate/up (GU, one or two tokens): a row group reads row n of the gate
// and of the up matrix in the same step and keeps silu(gate) * up, the decode
// form of the operation the skinny and prefill kernels fuse.  With rows split
// over S waves the gate and up slice sums meet in LDS separately and the SiLU
// is applied once they are whole.
//
// x is staged once per workgroup through LDS (coalesced 16-byte loads, one
// 144-byte slot per 128-byte pair chunk so the per-lane reads hit distinct
// banks) and kept in registers, permuted into the order the weight operands
// take it; the quantized values are multiplied as binary16 subnormals (the
// format policies FmtQ4 and FmtQ8 of gemv_formats.hpp), then a DPP wave sum
// and an exact power-of-two rescale.
#include "common.hpp"
#include "gemv_formats.hpp"
#include "q4_0.hpp"

namespace mote::q4_0 {
namespace {

constexpr int kStreamWaves = 8;
constexpr int kStreamThreads = kStreamWaves * kWave;
constexpr uint32_t kSlot = 144;

template <class F, int P, int S, int D, int MT, bool LAG, typename OutT, bool GU = false>
__global__ __launch_bounds__(kStreamThreads) void gemv_stream_kernel(const uint16_t* __restrict__ x,
                                                                     const uint8_t* __restrict__ w,
                                                                     const uint8_t* __restrict__ w_up,
                                                                     OutT* __restrict__ y, uint32_t N,
                                                                     uint32_t K, uint32_t total_groups) {
    // Gate/up with rows split over S waves (SPLIT_GU) carries the gate and up
    // sums separately through the cross-wave reduction and applies the SiLU
    // once they are whole.
    constexpr bool SPLIT_GU = GU && S > 1;
    constexpr int NW = GU ? 2 : 1;             // matrices read per row: gate (and up)
    constexpr int kGroups = kStreamWaves / S;  // row groups per workgroup
    extern __shared__ __attribute__((aligned(16))) uint8_t xs[];
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int slice = wave % S;
    const uint32_t npairs = K >> 6;
    const size_t row_bytes = static_cast<size_t>(npairs) * F::kPairBytes;
    // The S waves of a row group split each row into S slices of `span`
    // pairs; lane l of slice s owns pairs s*span + l + 64i (i < P).  Idle
    // slots are clamped to the last pair (a cached re-read) and dropped.
    const uint32_t span = (npairs + S - 1) / S;
    uint32_t pc[P], keep[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const uint32_t off = static_cast<uint32_t>(lane + 64 * i);
        const uint32_t pi = static_cast<uint32_t>(slice) * span + off;
        pc[i] = min(pi, npairs - 1);
        keep[i] = (off < span && pi < npairs) ? 0xFFFFFFFFu : 0u;  // bit mask: NaN-safe, branch-free drop
    }
    const uint32_t g = blockIdx.x * kGroups + static_cast<uint32_t>(wave / S);
    // rows g, g + T, ... (T row groups in the grid): count, and the last one
    // (prefetches past it re-read it, an L2 hit, so every load is
    // unconditional and vmcnt stays exact)
    const uint32_t nrows = g < N ? (N - 1 - g) / total_groups + 1 : 0;
    const uint32_t last = g < N ? g + (nrows - 1) * total_groups : N - 1;
    // Split rows reduce across waves through LDS behind barriers, so every
    // wave of the workgroup runs the trip count of its first row group (the
    // largest); the others compute clamped rows and store nothing.
    const uint32_t g0 = blockIdx.x * kGroups;
    const uint32_t trips = S == 1 ? nrows : (g0 < N ? (N - 1 - g0) / total_groups + 1 : 0);
    auto load_row = [&](uint32_t jj, uint32_t (&b)[NW * P][F::kDwords]) {
        const size_t offset = static_cast<size_t>(min(g + jj * total_groups, last)) * row_bytes;
#pragma unroll
        for (int mat = 0; mat < NW; ++mat) {
            const uint8_t* row = (mat == 0 ? w : w_up) + offset;
#pragma unroll
            for (int i = 0; i < P; ++i)
                F::load(row + static_cast<size_t>(pc[i]) * F::kPairBytes, b[mat * P + i]);
        }
    };

    // x chunk loads first (P S MT 16-byte chunks per thread; chunk c of the
    // [MT, K] activations is token c / (8 npairs), pair (c / 8) % npairs),
    // then the first D rows, and only then the LDS stores of x, so no row
    // load waits for x.
    constexpr int XC = P * S * MT;
    const uint32_t xchunks = npairs * 8 * MT;
    u32x4 xreg[XC];
    uint32_t xc[XC];
#pragma unroll
    for (int c = 0; c < XC; ++c) {
        xc[c] = min(static_cast<uint32_t>(tid + kStreamThreads * c), xchunks - 1);
        xreg[c] = reinterpret_cast<const u32x4*>(x)[xc[c]];
    }
    __builtin_amdgcn_sched_barrier(0);
    // Ring of D + 1 row buffers: row j + D is issued before row j is
    // computed, so D rows stay in flight behind the arithmetic (with LAG the
    // wave then waits for row j + 1 before issuing more; without it, D + 1
    // rows are in flight while it waits).
    constexpr int R = D + 1;
    uint32_t buf[R][NW * P][F::kDwords];
#pragma unroll
    for (int d = 0; d < D; ++d) load_row(static_cast<uint32_t>(d), buf[d]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < XC; ++c)
        *reinterpret_cast<u32x4*>(xs + (xc[c] >> 3) * kSlot + (xc[c] & 7) * 16) = xreg[c];
    __syncthreads();

    XPair xv[MT][P];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int s = 0; s < P; ++s) {
        uint32_t xr[32];
        const uint8_t* slot = xs + (static_cast<size_t>(m) * npairs + pc[s]) * kSlot;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(slot + i * 16);
            xr[4 * i + 0] = v.x; xr[4 * i + 1] = v.y; xr[4 * i + 2] = v.z; xr[4 * i + 3] = v.w;
        }
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            s0 = dot2(xr[i], kOnePair, s0);
            s1 = dot2(xr[16 + i], kOnePair, s1);
        }
        xv[m][s].c0 = F::kStart * s0;
        xv[m][s].c1 = F::kStart * s1;
        F::order_x(xr, xv[m][s]);
    }

    // Row sums stay in registers (lane j % 64 holds row j of this wave) and
    // are stored every 64 rows and at the end, so no store sits between the
    // pipelined loads.  Split rows first add the S slice sums through LDS
    // (after the x area).  The loop runs at least once and is unrolled by the
    // ring size, so slots are compile-time registers; steps past the last row
    // compute clamped rows and store nothing.
    float* red = reinterpret_cast<float*>(xs + static_cast<size_t>(npairs) * MT * kSlot);
    auto flush = [&](const float (&v)[MT], const float (&vu)[MT], uint32_t first, uint32_t count) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float t = v[m], tu = vu[m];
            if constexpr (S > 1) {
                red[wave * 64 + lane] = t;
                if constexpr (SPLIT_GU) red[kStreamThreads + wave * 64 + lane] = tu;
                __syncthreads();
                if (slice == 0) {
#pragma unroll
                    for (int r = 1; r < S; ++r) {
                        t += red[(wave + r) * 64 + lane];
                        if constexpr (SPLIT_GU) tu += red[kStreamThreads + (wave + r) * 64 + lane];
                    }
                }
                __syncthreads();
            }
            if constexpr (SPLIT_GU) t = silu(F::kFinal * t) * (F::kFinal * tu);
            if (slice == 0 && static_cast<uint32_t>(lane) < count)
                y[static_cast<size_t>(m) * N + g + (first + static_cast<uint32_t>(lane)) * total_groups] =
                    to_out<OutT>(GU ? t : F::kFinal * t);  // gate/up values are final here
        }
    };
    float mine[MT], mine_up[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) mine[m] = mine_up[m] = 0.0f;
    // The reference's per-element sum of this wave's share of row jj of `mat`
    // for token m, in the units of the dot chains (a row whose factored sum
    // is not finite; see gemv_formats.hpp).
    auto exact_share = [&](const uint8_t* mat, uint32_t jj, int m) {
        const uint8_t* row = mat + static_cast<size_t>(min(g + jj * total_groups, last)) * row_bytes;
        float e = 0.0f;
#pragma unroll  // pc and keep stay registers: no dynamic index
        for (int i = 0; i < P; ++i)
            if (keep[i] != 0u)
                e += F::exact(row + static_cast<size_t>(pc[i]) * F::kPairBytes,
                              x + static_cast<size_t>(m) * K + static_cast<size_t>(pc[i]) * 64u);
        return wave_sum(e) * (1.0f / F::kFinal);
    };
    uint32_t j = 0;
    do {
#pragma unroll
        for (int u = 0; u < R; ++u) {
            const uint32_t jj = j + static_cast<uint32_t>(u);
            load_row(jj + D, buf[(u + D) % R]);
            __builtin_amdgcn_sched_barrier(0);
            float part[MT], part_up[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) part[m] = part_up[m] = 0.0f;
#pragma unroll
            for (int i = 0; i < P; ++i) {
                if constexpr (MT == 1) {  // masks feed the dot chains directly: fewer live registers
                    part[0] += __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, F::dot(buf[u][i], xv[0][i])) & keep[i]);
                    if constexpr (GU)
                        part_up[0] += __builtin_bit_cast(
                            float, __builtin_bit_cast(uint32_t, F::dot(buf[u][P + i], xv[0][i])) & keep[i]);
                } else {
                    Unpacked wu;
                    F::unpack(buf[u][i], wu);
#pragma unroll
                    for (int m = 0; m < MT; ++m)
                        part[m] += __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, F::dot(wu, xv[m][i])) & keep[i]);
                    if constexpr (GU) {
                        Unpacked uu;
                        F::unpack(buf[u][P + i], uu);
#pragma unroll
                        for (int m = 0; m < MT; ++m)
                            part_up[m] += __builtin_bit_cast(
                                float, __builtin_bit_cast(uint32_t, F::dot(uu, xv[m][i])) & keep[i]);
                    }
                }
            }
            const bool mine_lane = jj < trips && static_cast<uint32_t>(lane) == (jj & 63u);
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                float s = wave_sum(part[m]);
                if (__builtin_expect(not_finite(s), 0)) s = exact_share(w, jj, m);  // wave-uniform
                if constexpr (GU) {
                    float su = wave_sum(part_up[m]);
                    if (__builtin_expect(not_finite(su), 0)) su = exact_share(w_up, jj, m);
                    if constexpr (SPLIT_GU)
                        mine_up[m] = mine_lane ? su : mine_up[m];
                    else
                        s = silu(F::kFinal * s) * (F::kFinal * su);
                }
                mine[m] = mine_lane ? s : mine[m];
            }
            if ((jj & 63u) == 63u && jj < trips)  // uniform over the workgroup
                flush(mine, mine_up, jj - 63u, nrows > jj - 63u ? min(nrows - (jj - 63u), 64u) : 0u);
            if constexpr (LAG) {
                // Row j + 1 arrives before row j + 1 + D is issued: D rows in
                // flight at any time, never D + 1.
                constexpr int kLater = 9 * NW * P * (D - 1);  // loads of rows j + 2 .. j + D
                __builtin_amdgcn_s_waitcnt((kLater & 0xF) | ((kLater >> 4) << 14) | 0x0F70);
            }
        }
        j += R;
    } while (j < trips);
    const uint32_t base = trips & ~63u;
    if (base < trips) flush(mine, mine_up, base, nrows > base ? nrows - base : 0u);
}

template <int P, int S, int D, int G, int MT = 1, bool LAG = true, class F = FmtQ4, bool GU = false>
hipError_t launch_gemv_stream(const Problem& p) {
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        return n;
    }();
    constexpr uint32_t kGroups = kStreamWaves / S;
    uint32_t groups = static_cast<uint32_t>(cus) * G;
    const uint32_t need = (p.N + kGroups - 1) / kGroups;  // no idle workgroups
    if (groups > need) groups = need;
    const uint32_t total_groups = groups * kGroups;
    const size_t lds = static_cast<size_t>(p.K / 64) * MT * kSlot + (S > 1 ? (GU ? 2 : 1) * kStreamThreads * sizeof(float) : 0);
    const dim3 grid(groups), block(kStreamThreads);
    if (p.out == OutType::F32) {
        hipLaunchKernelGGL((gemv_stream_kernel<F, P, S, D, MT, LAG, float, GU>), grid, block, lds, p.stream,
                           static_cast<const uint16_t*>(p.x), static_cast<const uint8_t*>(p.w),
                           static_cast<const uint8_t*>(p.w_up), static_cast<float*>(p.y), p.N, p.K,
                           total_groups);
    } else {
        hipLaunchKernelGGL((gemv_stream_kernel<F, P, S, D, MT, LAG, _Float16, GU>), grid, block, lds, p.stream,
                           static_cast<const uint16_t*>(p.x), static_cast<const uint8_t*>(p.w),
                           static_cast<const uint8_t*>(p.w_up), static_cast<_Float16*>(p.y), p.N, p.K,
                           total_groups);
    }
    return hipGetLastError();
}

// 5-16 tokens as passes of at most four tokens each (rows whole, S = 1, or
// split over S waves), every pass reading the weights once: for K with no
// split-K slicing (K % 1024 != 0, e.g. 3584, 11 008, 13 824), where the
// alternatives are the vector-ALU GEMV or the prefill tiles.
template <int S, class F>
hipError_t launch_gemv_stream_groups(const Problem& p) {
    const size_t out_bytes = p.out == OutType::F32 ? 4 : 2;
    for (uint32_t m0 = 0; m0 < p.M;) {
        const uint32_t mt = p.M - m0 < 4u ? p.M - m0 : 4u;
        Problem q = p;
        q.M = mt;
        q.x = static_cast<const uint16_t*>(p.x) + static_cast<size_t>(m0) * p.K;
        q.y = static_cast<uint8_t*>(p.y) + static_cast<size_t>(m0) * p.N * out_bytes;
        hipError_t e;
        switch (mt) {
            case 4: e = launch_gemv_stream<1, S, 1, 1, 4, false, F>(q); break;
            case 3: e = launch_gemv_stream<1, S, 1, 1, 3, false, F>(q); break;
            case 2: e = launch_gemv_stream<1, S, 1, 1, 2, false, F>(q); break;
            default: e = launch_gemv_stream<1, S, 1, 1, 1, false, F>(q); break;
        }
        if (e != hipSuccess) return e;
        m0 += mt;
    }
    return hipSuccess;
}

// p0 = 64-pair capacity of a row (K <= 4096 p0), p1 = rows in flight,
// p2 = workgroups per CU.
#define MOTE_STREAM(D, G) \
    Variant{"stream_d" #D "_g" #G, Kind::GemvStream, 1, D, G, &launch_gemv_stream<1, 1, D, G>}
#define MOTE_STREAM_Q(D, G) \
    Variant{"stream_d" #D "q_g" #G, Kind::GemvStream, 1, D, G, &launch_gemv_stream<1, 1, D, G, 1, false>}
#define MOTE_STREAM_S(S, D, G) \
    Variant{"stream_s" #S "_d" #D "_g" #G, Kind::GemvStream, S, D, G, &launch_gemv_stream<1, S, D, G>}
#define MOTE_STREAM_SQ(S, D, G)                                              \
    Variant{"stream_s" #S "_d" #D "q_g" #G, Kind::GemvStream, S, D, G,       \
            &launch_gemv_stream<1, S, D, G, 1, false>}
#define MOTE_STREAM_M(MT, D, G)                                                          \
    Variant{"stream_m" #MT "_d" #D "_g" #G, Kind::GemvStream, 1, D, G,                  \
            &launch_gemv_stream<1, 1, D, G, MT>, MT}
#define MOTE_Q8(NAME, S, G) \
    Variant{"q8_stream_" NAME, Kind::Q8Stream, S, 1, G, &launch_gemv_stream<1, S, 1, G, 1, true, FmtQ8>}
#define MOTE_Q8_M(MT, G)                                                             \
    Variant{"q8_stream_m" #MT "_d1q_g" #G, Kind::Q8Stream, 1, 1, G,                \
            &launch_gemv_stream<1, 1, 1, G, MT, false, FmtQ8>, MT}
#define MOTE_Q8_SM(S, MT)                                                               \
    Variant{"q8_stream_s" #S "_m" #MT "_d1q_g1", Kind::Q8Stream, S, 1, 1,                \
            &launch_gemv_stream<1, S, 1, 1, MT, false, FmtQ8>, MT}
#define MOTE_STREAM_GU(P, G)                                                             \
    Variant{"gateup_stream_p" #P "_d1_g" #G, Kind::GateUpStream, P, 1, G,               \
            &launch_gemv_stream<P, 1, 1, G, 1, true, FmtQ4, true>}
#define MOTE_STREAM_SMQ(S, MT, G)                                                        \
    Variant{"stream_s" #S "_m" #MT "_d1q_g" #G, Kind::GemvStream, S, 1, G,              \
            &launch_gemv_stream<1, S, 1, G, MT, false>, MT}
#define MOTE_STREAM_GU_SMQ(S, MT)                                                        \
    Variant{"gateup_stream_s" #S "_m" #MT "_d1q_g1", Kind::GateUpStream, S, 1, 1,        \
            &launch_gemv_stream<1, S, 1, 1, MT, false, FmtQ4, true>, MT}
#define MOTE_STREAM_GU_MQ(P, MT)                                                         \
    Variant{"gateup_stream_p" #P "_m" #MT "_d1q_g1", Kind::GateUpStream, P, 1, 1,       \
            &launch_gemv_stream<P, 1, 1, 1, MT, false, FmtQ4, true>, MT}
#define MOTE_STREAM_MQ(MT, D, G)                                                         \
    Variant{"stream_m" #MT "_d" #D "q_g" #G, Kind::GemvStream, 1, D, G,                 \
            &launch_gemv_stream<1, 1, D, G, MT, false>, MT}

// "q" variants queue row j + 1 + D while waiting for row j + 1.  The table
// holds the forms the dispatch heuristic picks plus the measured alternatives
// it is compared with (two rows in flight, the other queueing form, one or
// two workgroups per CU, three and four tokens per row read).
const Variant kStream[] = {
    MOTE_STREAM(1, 1), MOTE_STREAM(2, 1), MOTE_STREAM(1, 2),
    MOTE_STREAM_Q(1, 1), MOTE_STREAM_Q(1, 2),
    MOTE_STREAM_S(2, 1, 1), MOTE_STREAM_S(2, 1, 2), MOTE_STREAM_SQ(4, 1, 1), MOTE_STREAM_SQ(4, 1, 2),
    MOTE_STREAM_S(8, 1, 1), MOTE_STREAM_S(8, 1, 2),
    MOTE_STREAM_M(3, 1, 1), MOTE_STREAM_M(4, 1, 1), MOTE_STREAM_MQ(2, 1, 1),
    MOTE_STREAM_SMQ(2, 2, 1), MOTE_STREAM_SMQ(4, 2, 1), MOTE_STREAM_SMQ(8, 2, 1),
    MOTE_STREAM_SMQ(2, 3, 1), MOTE_STREAM_SMQ(4, 3, 1), MOTE_STREAM_SMQ(2, 4, 1), MOTE_STREAM_SMQ(4, 4, 1),
    MOTE_Q8("d1_g1", 1, 1), MOTE_Q8("d1_g2", 1, 2), MOTE_Q8("s2_d1_g1", 2, 1), MOTE_Q8("s4_d1_g1", 4, 1),
    MOTE_Q8("s8_d1_g1", 8, 1),
    MOTE_Q8_SM(2, 2), MOTE_Q8_SM(4, 2), MOTE_Q8_SM(8, 2), MOTE_Q8_SM(2, 3), MOTE_Q8_SM(4, 3), MOTE_Q8_SM(2, 4), MOTE_Q8_SM(4, 4),
    // tokens = -4: 5-16 tokens in passes of four
    Variant{"q8_stream_s2_m4x_d1q_g1", Kind::Q8Stream, 2, 1, 1, &launch_gemv_stream_groups<2, FmtQ8>, -4},
    Variant{"q8_stream_s4_m4x_d1q_g1", Kind::Q8Stream, 4, 1, 1, &launch_gemv_stream_groups<4, FmtQ8>, -4},
    Variant{"stream_m4x_d1q_g1", Kind::GemvStream, 1, 1, 1, &launch_gemv_stream_groups<1, FmtQ4>, -4},
    Variant{"stream_s2_m4x_d1q_g1", Kind::GemvStream, 2, 1, 1, &launch_gemv_stream_groups<2, FmtQ4>, -4},
    Variant{"stream_s4_m4x_d1q_g1", Kind::GemvStream, 4, 1, 1, &launch_gemv_stream_groups<4, FmtQ4>, -4}, MOTE_Q8_M(2, 1), MOTE_Q8_M(4, 1),
    MOTE_STREAM_GU(1, 1), MOTE_STREAM_GU(1, 2),
    MOTE_STREAM_GU_MQ(1, 2), MOTE_STREAM_GU_SMQ(2, 2), MOTE_STREAM_GU_SMQ(4, 2), MOTE_STREAM_GU_SMQ(8, 2),
    MOTE_STREAM_GU_SMQ(2, 1), MOTE_STREAM_GU_SMQ(4, 1), MOTE_STREAM_GU_SMQ(8, 1),
    MOTE_STREAM_GU_SMQ(2, 3), MOTE_STREAM_GU_SMQ(4, 3),
};

#undef MOTE_STREAM
#undef MOTE_STREAM_S
#undef MOTE_STREAM_M
#undef MOTE_STREAM_Q
#undef MOTE_STREAM_SQ
#undef MOTE_STREAM_MQ
#undef MOTE_STREAM_GU_MQ
#undef MOTE_STREAM_GU_SMQ
#undef MOTE_STREAM_SMQ
#undef MOTE_Q8_SM
#undef MOTE_Q8
#undef MOTE_Q8_M
#undef MOTE_STREAM_GU

}  // namespace

const Variant* gemv_stream_variants(int* count) {
    *count = static_cast<int>(sizeof(kStream) / sizeof(kStream[0]));
    return kStream;
}

// One token (or exactly the variant's token count), K a multiple of 64 and at
// most 4096 per 64-pair slot of a row, x 16-byte and w (and the up matrix of a
// gate/up) dword aligned.
bool gemv_stream_supports(const Variant& v, const Problem& p) {
    if (v.tokens < 0) {  // passes of -tokens tokens: 5-16 tokens, each pass as that many
        if (p.M < 5 || p.M > 16) return false;
        Variant pass = v;
        pass.tokens = -v.tokens;
        Problem q = p;
        q.M = static_cast<uint32_t>(pass.tokens);
        return gemv_stream_supports(pass, q);
    }
    const uint32_t tokens = v.tokens > 0 ? static_cast<uint32_t>(v.tokens) : 1u;
    const bool up_ok = v.kind != Kind::GateUpStream ||
                       (p.w_up != nullptr && reinterpret_cast<uintptr_t>(p.w_up) % 4 == 0);
    // the activations of every token (and the split-row sums) fit one
    // workgroup's 160 KB of LDS
    const uint64_t lds = static_cast<uint64_t>(p.K / 64) * tokens * kSlot + 2 * kStreamThreads * sizeof(float);
    return p.M == tokens && p.K % 64 == 0 && p.K > 0 && p.K <= 4096u * static_cast<uint32_t>(v.p0) &&
           lds <= 160u * 1024u && reinterpret_cast<uintptr_t>(p.w) % 4 == 0 &&
           reinterpret_cast<uintptr_t>(p.x) % 16 == 0 && up_ok;
}

}  // namespace mote::q4_0

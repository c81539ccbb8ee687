// Decode GEMV over GGML Q4_0 and Q8_0 for K a multiple of 256, with the weight
// rows streamed through a per-wave LDS ring by CDNA4's direct-to-LDS loads:
// whole rows for K up to 4096 (one token; Q8_0 also two or three tokens per
// row read), rows split over 2, 4 or 8 waves past that (one token).
//
// Computes y[m, n] = sum_k x[m, k] * w[n, k] for f16 x [M, K] and quantized
// w [N, K], the operation of crates/mote-backend-hip/src/
// quantized_linear.hip:13-52 (oracle crates/mote-reference/src/
// quantized.rs:89-144; Q8_0 decode at :191-195).
//
// Why: a wave that loads its lanes' 36-byte block pairs directly issues three
// strided instructions per row, each touching every cache line of the row, so
// the loads cannot be non-temporal (the second and third would re-fetch lines
// the first evicted).  Measured on MI355X, pure reads of the 33 MB up/gate
// matrix in the decode's row order take 6.3 us with pair loads and 5.9 us
// with coalesced non-temporal 16-byte loads.  Here every row is read as
// consecutive 16-byte chunks (lane l takes chunks l, 64 + l, ...), each line
// once, non-temporally, straight into the wave's LDS ring
// (global_load_lds_dwordx4), and each lane then reads its pair from LDS
// (nine dwords at a 36-byte stride: distinct banks).  x also arrives by a
// direct-to-LDS load, issued before any weight load and waited for with the
// first rows in flight.  The arithmetic is the streaming GEMV's (q4_0_gemv
// _stream.hip: nibbles as binary16 subnormals, v_dot2_f32_f16, DPP wave sum),
// so the two kernels agree bit for bit.
//
// Grid: one workgroup of 8 waves per CU (more measured slower: the LDS ring of
// 16 waves per CU puts too many rows in flight); wave g walks rows g, g + T,
// ... (T waves in the grid).  R ring slots, D rows in flight ahead of the
// one being computed, none past the wave's last row.  Measured on MI355X (K = 4096): N = 14336 7.27 us
// (the pair-load kernel: 7.62), 11008 6.23 (7.07), 6144 4.62 (5.14), 4096
// 3.90 (4.22), 1024 3.12 (3.51).
#include "common.hpp"
#include "gemv_formats.hpp"
#include "gemv_lds.hpp"
#include "q4_0.hpp"

namespace mote::q4_0 {
namespace {

// F: the weight format (FmtQ4: 36-byte Q4_0 block pairs, FmtQ8: 68-byte Q8_0
// pairs); MT: tokens, every row read once for all of them.  The body is
// gemv_lds_body (gemv_lds.hpp).
template <class F, int MT, int R, int D, int LOADS, typename OutT>
__global__ __launch_bounds__(kThreads) void gemv_lds_kernel(const uint16_t* __restrict__ x,
                                                           const uint8_t* __restrict__ w, OutT* __restrict__ y,
                                                           uint32_t N, uint32_t K, uint32_t total_groups) {
    NoTimeline tl;
    gemv_lds_body<F, MT, R, D, LOADS, OutT>(x, w, y, N, K, total_groups, tl);
}

// LDS slot of a slice of `span` pairs: the 16-byte chunks that overlap it
// wherever it starts (a multiple of 4 bytes into a chunk).
__host__ __device__ constexpr uint32_t slot_size(uint32_t span, uint32_t pair_bytes) {
    return (span * pair_bytes + 15u) / 16u * 16u + 16u;
}

// Load instructions per slice of a row split over s waves: enough for the
// widest slice, and 0 (unsupported) unless every slice's last instruction
// keeps at least one lane (the wait counts assume LOADS loads per row, and the
// other instructions load whole).
inline uint32_t split_loads(uint32_t s, uint32_t k, uint32_t pair_bytes) {
    const uint32_t npairs = k / 64, span = (npairs + s - 1) / s;
    uint32_t lo = 0xFFFFFFFFu, hi = 0;
    for (uint32_t i = 0; i < s; ++i) {
        if (i * span >= npairs) return 0;
        const uint32_t b0 = i * span * pair_bytes, count = npairs - i * span < span ? npairs - i * span : span;
        const uint32_t chunks = (b0 + count * pair_bytes + 15u) / 16u - b0 / 16u;
        lo = chunks < lo ? chunks : lo;
        hi = chunks > hi ? chunks : hi;
    }
    const uint32_t loads = (hi + 63u) / 64u;
    return loads >= 1 && loads <= 5 && lo > 64u * (loads - 1) ? loads : 0;
}

// Dynamic LDS of the split-row kernel: the waves' rings, then x in 8 KB steps.
__host__ __device__ constexpr size_t split_lds_bytes(uint32_t s, uint32_t r, uint32_t k, uint32_t pair_bytes) {
    return static_cast<size_t>(kWaves) * r * slot_size((k / 64 + s - 1) / s, pair_bytes) + (k + 4095u) / 4096u * 8192u;
}

// Rows split over S waves (K past 4096, up to about 4096 S): wave w of a
// workgroup reads slice w % S of its row group's rows -- pairs [s span,
// min((s + 1) span, K / 64)) with span = ceil(K / (64 S)), the pair
// assignment of the split-row streaming GEMV -- through its own ring, and
// lane l owns pair l of the slice.  A slice starts 36 s span bytes into a row
// (rows start on 16-byte boundaries, K % 256 == 0), so its loads cover the
// 16-byte chunks that overlap it and its pairs sit (36 s span) % 16 bytes
// into the ring slot.  x is staged once per workgroup in LDS by direct-to-LDS
// loads (thread t loads 16-byte chunks t, t + 512, ..., clamped, into 8 KB
// steps), issued before the first rows; each lane then reads its pair's 128
// bytes (measured on MI355X at 14336 x 4096: 7.85 us, against 8.69 us with
// every lane loading its pair's x into registers, twice the L2 traffic).
// The slice sums are added in slice order through LDS, as in the streaming
// GEMV, so the two agree bit for bit; that addition sits behind workgroup
// barriers, so every wave runs the row count of its workgroup's first row
// group (the largest), and a group with one row fewer re-reads its last row
// once and does not store it.
template <class F, int S, int R, int D, int LOADS, typename OutT>
__global__ __launch_bounds__(kThreads) void gemv_lds_split_kernel(const uint16_t* __restrict__ x,
                                                                 const uint8_t* __restrict__ w,
                                                                 OutT* __restrict__ y, uint32_t N, uint32_t K,
                                                                 uint32_t total_groups) {
    static_assert(S == 2 || S == 4 || S == 8, "whole row groups per workgroup");
    static_assert(D >= 1 && D <= 3 && D < R, "the ring holds the rows in flight and the one computed");
    constexpr uint32_t kGroups = kWaves / S;
    // [waves][R][slot bytes], then x in 8 KB steps
    extern __shared__ __attribute__((aligned(16))) uint8_t ring_lds[];
    __shared__ float red[kThreads];  // slice sums of 64 rows
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const uint32_t slice = static_cast<uint32_t>(wave) % S;
    const uint32_t npairs = K >> 6;
    const uint32_t span = (npairs + S - 1) / S;
    const uint32_t first_pair = slice * span;
    const uint32_t count = min(span, npairs - first_pair);  // >= 1: every slice holds pairs
    const size_t row_bytes = static_cast<size_t>(npairs) * F::kPairBytes;  // a multiple of 16
    const uint32_t b0 = first_pair * F::kPairBytes;
    const uint32_t c0 = b0 >> 4;
    const uint32_t chunks = (b0 + count * F::kPairBytes + 15u) / 16u - c0;
    const uint32_t slot_bytes = slot_size(span, F::kPairBytes);
    uint8_t* ring = ring_lds + static_cast<uint32_t>(wave) * R * slot_bytes;
    const uint32_t g = blockIdx.x * kGroups + static_cast<uint32_t>(wave) / S;
    const uint32_t nrows = g < N ? (N - 1 - g) / total_groups + 1 : 0;
    const uint32_t last = g < N ? g + (nrows - 1) * total_groups : N - 1;
    // the grid has no workgroup without a row: its first group's g < N
    const uint32_t trips = (N - 1 - blockIdx.x * kGroups) / total_groups + 1;
    const uint32_t pc = min(static_cast<uint32_t>(lane), count - 1);
    const uint32_t keep = static_cast<uint32_t>(lane) < count ? 0xFFFFFFFFu : 0u;  // NaN-safe drop of idle lanes
    const uint8_t* wslice = w + 16u * c0;

    // Chunks of row jj's slice (jj < trips) into ring slot `slot`; the last
    // instruction's lanes past the slice idle (lane 0 always loads).
    auto load_row = [&](uint32_t jj, uint32_t slot) {
        const uint8_t* src = wslice + static_cast<size_t>(min(g + jj * total_groups, last)) * row_bytes;
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const uint32_t c = 64u * static_cast<uint32_t>(i) + static_cast<uint32_t>(lane);
            if (i + 1 < LOADS || c < chunks)
                __builtin_amdgcn_global_load_lds(src + 16u * c, (lds_ptr)(ring + slot * slot_bytes + 1024u * i), 16,
                                                 0, 2 /* non-temporal */);
        }
    };
    auto wait_rows = [&](uint32_t rows) {
        if (rows >= 3 && D >= 3) __builtin_amdgcn_s_waitcnt(vm_wait(LOADS * 3));
        else if (rows == 2 && D >= 2) __builtin_amdgcn_s_waitcnt(vm_wait(LOADS * 2));
        else if (rows == 1) __builtin_amdgcn_s_waitcnt(vm_wait(LOADS));
        else __builtin_amdgcn_s_waitcnt(vm_wait(0));
    };

    // x first, then the first rows; loads retire in order, so once only those
    // rows are outstanding this wave's x chunks have landed, and after the
    // barrier every wave's have.
    const uint32_t xsteps = (K + 4095u) / 4096u;
    uint8_t* xs = ring_lds + kWaves * R * slot_bytes;
    for (uint32_t i = 0; i < xsteps; ++i) {
        const uint32_t c = min(swizzled_chunk(512u * i + static_cast<uint32_t>(tid)), K / 8u - 1u);
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t*>(x) + 16u * c,
                                         (lds_ptr)(xs + 8192u * i + 1024u * static_cast<uint32_t>(wave)), 16, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int d = 0; d < D; ++d)
        if (static_cast<uint32_t>(d) < trips) load_row(static_cast<uint32_t>(d), static_cast<uint32_t>(d));
    __builtin_amdgcn_sched_barrier(0);
    wait_rows(trips < static_cast<uint32_t>(D) ? trips : static_cast<uint32_t>(D));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    XPair xv;
    {
        uint32_t xr[32];
        const uint32_t xp = first_pair + pc;
        const uint8_t* xslot = xs + xp * 128u;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(xslot + ((static_cast<uint32_t>(i) + xp) & 7u) * 16u);
            xr[4 * i + 0] = v.x; xr[4 * i + 1] = v.y; xr[4 * i + 2] = v.z; xr[4 * i + 3] = v.w;
        }
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            s0 = dot2(xr[i], kOnePair, s0);
            s1 = dot2(xr[16 + i], kOnePair, s1);
        }
        xv.c0 = F::kStart * s0;
        xv.c1 = F::kStart * s1;
        F::order_x(xr, xv);
    }

    // Lane j % 64 holds the slice sum of row j; every 64 rows and at the end
    // slice 0 adds the other slices' sums (in slice order) and stores.
    float mine = 0.0f;
    auto flush = [&](uint32_t first, uint32_t n) {
        red[tid] = mine;
        __syncthreads();
        float t = mine;
        if (slice == 0) {
#pragma unroll
            for (int r = 1; r < S; ++r) t += red[(wave + r) * 64 + lane];
        }
        __syncthreads();
        if (slice == 0 && static_cast<uint32_t>(lane) < n)
            y[g + (first + static_cast<uint32_t>(lane)) * total_groups] = to_out<OutT>(F::kFinal * t);
    };
    const uint32_t pair_offset = (b0 & 15u) + pc * F::kPairBytes;
    for (uint32_t j = 0; j < trips; ++j) {
        if (j + D < trips) {
            load_row(j + D, (j + D) % R);
            __builtin_amdgcn_s_waitcnt(vm_wait(LOADS * D));
        } else {
            wait_rows(trips - 1 - j);
        }
        const uint32_t* pr = reinterpret_cast<const uint32_t*>(ring + (j % R) * slot_bytes + pair_offset);
        uint32_t raw[F::kDwords];
#pragma unroll
        for (int i = 0; i < F::kDwords; ++i) raw[i] = pr[i];
        const float part = 0.0f + __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, F::dot(raw, xv)) & keep);
        float s = wave_sum(part);
        if (__builtin_expect(not_finite(s), 0)) {  // wave-uniform: the reference's per-element sum of the slice
            const uint32_t pi = first_pair + pc;
            const uint8_t* pair = w + static_cast<size_t>(min(g + j * total_groups, last)) * row_bytes + pi * F::kPairBytes;
            const float e = keep != 0u ? F::exact(pair, x + pi * 64u) : 0.0f;
            s = wave_sum(e) * (1.0f / F::kFinal);
        }
        mine = static_cast<uint32_t>(lane) == (j & 63u) ? s : mine;
        if ((j & 63u) == 63u) {  // uniform over the workgroup
            const uint32_t first = j - 63u;
            flush(first, nrows > first ? min(nrows - first, 64u) : 0u);
        }
    }
    const uint32_t base = trips & ~63u;
    if (base < trips) flush(base, nrows > base ? nrows - base : 0u);
}

template <class F, int MT, int R, int D>
hipError_t launch_gemv_lds(const Problem& p) {
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        return n;
    }();
    const uint32_t row_bytes = p.K / 64 * F::kPairBytes;
    const uint32_t loads = (row_bytes / 16 + 63) / 64;
    uint32_t groups = static_cast<uint32_t>(cus);
    const uint32_t need = (p.N + kWaves - 1) / kWaves;  // no workgroup without a row
    if (groups > need) groups = need;
    const size_t lds = static_cast<size_t>(kWaves) * R * row_bytes;
    const dim3 grid(groups), block(kThreads);
    const auto* x = static_cast<const uint16_t*>(p.x);
    const auto* w = static_cast<const uint8_t*>(p.w);
    const uint32_t total = groups * kWaves;
#define MOTE_LDS_LAUNCH(L)                                                                                       \
    do {                                                                                                         \
        if (p.out == OutType::F32)                                                                               \
            hipLaunchKernelGGL((gemv_lds_kernel<F, MT, R, D, L, float>), grid, block, lds, p.stream, x, w,      \
                               static_cast<float*>(p.y), p.N, p.K, total);                                     \
        else                                                                                                     \
            hipLaunchKernelGGL((gemv_lds_kernel<F, MT, R, D, L, _Float16>), grid, block, lds, p.stream, x, w,   \
                               static_cast<_Float16*>(p.y), p.N, p.K, total);                                  \
    } while (0)
    switch (loads) {
        case 1: MOTE_LDS_LAUNCH(1); break;
        case 2: MOTE_LDS_LAUNCH(2); break;
        case 3: MOTE_LDS_LAUNCH(3); break;
        case 4:
        case 5:  // Q8_0 rows past 3584 elements
            if constexpr (F::kPairBytes > kPairBytes) {
                if (loads == 4) MOTE_LDS_LAUNCH(4);
                else MOTE_LDS_LAUNCH(5);
                break;
            } else {
                return hipErrorInvalidValue;
            }
        default: return hipErrorInvalidValue;
    }
#undef MOTE_LDS_LAUNCH
    return hipGetLastError();
}

template <class F, int S, int R, int D, int G>
hipError_t launch_gemv_lds_split(const Problem& p) {
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        return n;
    }();
    constexpr uint32_t kGroups = kWaves / S;
    const uint32_t loads = split_loads(S, p.K, F::kPairBytes);
    uint32_t groups = static_cast<uint32_t>(cus) * G;
    const uint32_t need = (p.N + kGroups - 1) / kGroups;  // no workgroup without a row
    if (groups > need) groups = need;
    const size_t lds = split_lds_bytes(S, R, p.K, F::kPairBytes);
    const dim3 grid(groups), block(kThreads);
    const auto* x = static_cast<const uint16_t*>(p.x);
    const auto* w = static_cast<const uint8_t*>(p.w);
    const uint32_t total = groups * kGroups;
#define MOTE_LDS_LAUNCH(L)                                                                                      \
    do {                                                                                                        \
        if (p.out == OutType::F32)                                                                              \
            hipLaunchKernelGGL((gemv_lds_split_kernel<F, S, R, D, L, float>), grid, block, lds, p.stream, x, w,   \
                               static_cast<float*>(p.y), p.N, p.K, total);                                    \
        else                                                                                                    \
            hipLaunchKernelGGL((gemv_lds_split_kernel<F, S, R, D, L, _Float16>), grid, block, lds, p.stream, x, w, \
                               static_cast<_Float16*>(p.y), p.N, p.K, total);                                 \
    } while (0)
    switch (loads) {
        case 1: MOTE_LDS_LAUNCH(1); break;
        case 2: MOTE_LDS_LAUNCH(2); break;
        case 3: MOTE_LDS_LAUNCH(3); break;
        case 4:
        case 5:  // Q8_0 slices past 42 pairs
            if constexpr (F::kPairBytes > kPairBytes) {
                if (loads == 4) MOTE_LDS_LAUNCH(4);
                else MOTE_LDS_LAUNCH(5);
                break;
            } else {
                return hipErrorInvalidValue;
            }
        default: return hipErrorInvalidValue;
    }
#undef MOTE_LDS_LAUNCH
    return hipGetLastError();
}

// p0 = ring slots, p1 = rows in flight, p2 = waves per row (0: one);
// tokens = the exact M of the multi-token variants.
const Variant kLds[] = {
    Variant{"rowlds_r2d1", Kind::GemvLds, 2, 1, 0, &launch_gemv_lds<FmtQ4, 1, 2, 1>},
    Variant{"rowlds_r3d1", Kind::GemvLds, 3, 1, 0, &launch_gemv_lds<FmtQ4, 1, 3, 1>},
    Variant{"rowlds_r3d2", Kind::GemvLds, 3, 2, 0, &launch_gemv_lds<FmtQ4, 1, 3, 2>},
    // two tokens, each row read once for both (2 x 4096 x 4096 / 6144 / 14336
    // in 4.25 / 5.11 / 8.37 us against 4.94 on the streaming GEMV and 6.22 /
    // 8.97 on the skinny tiles; three tokens measured slower at N = 14336)
    Variant{"rowlds_m2_r2d1", Kind::GemvLds, 2, 1, 0, &launch_gemv_lds<FmtQ4, 2, 2, 1>, 2},
    Variant{"rowlds_m3_r2d1", Kind::GemvLds, 2, 1, 0, &launch_gemv_lds<FmtQ4, 3, 2, 1>, 3},
    Variant{"rowlds_m4_r2d1", Kind::GemvLds, 2, 1, 0, &launch_gemv_lds<FmtQ4, 4, 2, 1>, 4},
#define MOTE_LDS_Q8(MT, R, D)                                                          \
    Variant{MT == 1 ? "q8_rowlds_r" #R "d" #D : "q8_rowlds_m" #MT "_r" #R "d" #D, Kind::Q8Lds, R, D, 0,     \
            &launch_gemv_lds<FmtQ8, MT, R, D>, MT}
    MOTE_LDS_Q8(1, 2, 1), MOTE_LDS_Q8(1, 3, 2), MOTE_LDS_Q8(2, 2, 1), MOTE_LDS_Q8(2, 3, 2), MOTE_LDS_Q8(3, 2, 1),
    MOTE_LDS_Q8(4, 2, 1),
#undef MOTE_LDS_Q8
#define MOTE_LDS_SPLIT(S, R, D, G) \
    Variant{"rowlds_s" #S "_r" #R "d" #D "_g" #G, Kind::GemvLds, R, D, S, &launch_gemv_lds_split<FmtQ4, S, R, D, G>}
    MOTE_LDS_SPLIT(2, 3, 2, 1), MOTE_LDS_SPLIT(4, 2, 1, 1), MOTE_LDS_SPLIT(4, 3, 2, 1), MOTE_LDS_SPLIT(4, 4, 3, 1),
    MOTE_LDS_SPLIT(8, 3, 2, 1),
#undef MOTE_LDS_SPLIT
#define MOTE_LDS_SPLIT_Q8(S, R, D)                                            \
    Variant{"q8_rowlds_s" #S "_r" #R "d" #D, Kind::Q8Lds, R, D, S, &launch_gemv_lds_split<FmtQ8, S, R, D, 1>}
    MOTE_LDS_SPLIT_Q8(2, 2, 1), MOTE_LDS_SPLIT_Q8(4, 2, 1), MOTE_LDS_SPLIT_Q8(4, 3, 2), MOTE_LDS_SPLIT_Q8(8, 2, 1),
#undef MOTE_LDS_SPLIT_Q8
};

}  // namespace

const Variant* gemv_lds_variants(int* count) {
    *count = static_cast<int>(sizeof(kLds) / sizeof(kLds[0]));
    return kLds;
}

// The variant's tokens (one, or 2-4 for the multi-token rings), K a multiple
// of 256 (rows start on 16-byte boundaries) up to 4096 (one pair per lane),
// or one token with rows split over S waves, up to 64 pairs per slice, every
// slice non-empty; the rings and x within the workgroup's 160 KB of LDS;
// weights and x 16-byte aligned (the direct-to-LDS loads move aligned 16-byte
// chunks).
bool gemv_lds_supports(const Variant& v, const Problem& p) {
    const uint32_t tokens = v.tokens > 0 ? static_cast<uint32_t>(v.tokens) : 1u;
    if (p.M != tokens || p.K % 256 != 0 || p.K == 0 || p.w_up != nullptr ||
        reinterpret_cast<uintptr_t>(p.w) % 16 != 0 || reinterpret_cast<uintptr_t>(p.x) % 16 != 0)
        return false;
    const uint32_t pair_bytes = v.kind == Kind::Q8Lds ? 68u : kPairBytes;
    if (v.p2 <= 1)
        return p.K <= kMaxK && static_cast<size_t>(kWaves) * v.p0 * (p.K / 64 * pair_bytes) +
                                       tokens * kMaxK * 2 <= 160u * 1024u;
    const uint32_t s = static_cast<uint32_t>(v.p2), npairs = p.K / 64, span = (npairs + s - 1) / s;
    return tokens == 1 && span <= 64 && (s - 1) * span < npairs && split_loads(s, p.K, pair_bytes) != 0 &&
           split_lds_bytes(s, static_cast<uint32_t>(v.p0), p.K, pair_bytes) + kThreads * sizeof(float) <=
               160u * 1024u;
}

}  // namespace mote::q4_0

// Decode GEMV (M = 1) over GGML Q4_0 for K a multiple of 256 up to 4096, with
// the weight rows streamed through a per-wave LDS ring by CDNA4's
// direct-to-LDS loads.
//
// Computes y[n] = sum_k x[k] * w[n, k] for f16 x [1, K] and Q4_0 w [N, K], the
// operation of crates/mote-backend-hip/src/quantized_linear.hip:13-52 (oracle
// crates/mote-reference/src/quantized.rs:89-144) at one token.
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
#include "q4_0.hpp"

namespace mote::q4_0 {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kWave;
constexpr uint32_t kSubLo = 0x000F000Fu;  // low nibbles of bytes 0 and 2: n * 2^-24
constexpr uint32_t kSubHi = 0x00F000F0u;  // high nibbles of bytes 0 and 2: n * 2^-20
constexpr uint32_t kMaxK = 4096;
typedef __attribute__((address_space(3))) void* lds_ptr;

__device__ __forceinline__ uint32_t pick(const uint32_t* x, int a, int b) {
    const uint32_t lo = (a & 1) ? 0x0302u : 0x0100u;
    const uint32_t hi = (b & 1) ? 0x07060000u : 0x05040000u;
    return __builtin_amdgcn_perm(x[b >> 1], x[a >> 1], hi | lo);
}

// x of a pair in the order of the nibble operands, and the start values of
// the two blocks' sums (-8 2^-20 times the block's sum of x).
struct XPair {
    uint32_t xp[32];
    float c0, c1;
};

__device__ __forceinline__ void order_x(const uint32_t (&xr)[32], XPair& xv) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const int base = (q < 4) ? 0 : 32;
        const int e0 = base + pair_byte_element(q, 0), e1 = base + pair_byte_element(q, 1);
        const int e2 = base + pair_byte_element(q, 2), e3 = base + pair_byte_element(q, 3);
        xv.xp[4 * q + 0] = pick(xr, e0 + 16, e2 + 16);  // hi02
        xv.xp[4 * q + 1] = pick(xr, e0, e2);            // lo02
        xv.xp[4 * q + 2] = pick(xr, e1, e3);            // lo13
        xv.xp[4 * q + 3] = pick(xr, e1 + 16, e3 + 16);  // hi13
    }
}

// sum_k x_k (n_k - 8) d of the two blocks of a pair, divided by 2^20.
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

// LOADS: 16-byte chunks of a row / 64, rounded up (1 for K <= 1792, 2 up to
// 3584, 3 up to 4096).
template <int R, int D, int LOADS, typename OutT>
__global__ __launch_bounds__(kThreads) void gemv_lds_kernel(const uint16_t* __restrict__ x,
                                                           const uint8_t* __restrict__ w, OutT* __restrict__ y,
                                                           uint32_t N, uint32_t K, uint32_t total_groups) {
    static_assert(D >= 1 && D <= 3 && D < R, "the ring holds the rows in flight and the one computed");
    extern __shared__ __attribute__((aligned(16))) uint8_t ring_lds[];     // [waves][R][row bytes]
    __shared__ __attribute__((aligned(16))) uint8_t xs[kMaxK * 2];        // x, contiguous
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const uint32_t npairs = K >> 6;
    const uint32_t row_bytes = npairs * kPairBytes;  // a multiple of 16: K % 256 == 0
    const uint32_t chunks = row_bytes >> 4;
    uint8_t* ring = ring_lds + static_cast<uint32_t>(wave) * R * row_bytes;
    const uint32_t g = blockIdx.x * kWaves + static_cast<uint32_t>(wave);
    const uint32_t nrows = g < N ? (N - 1 - g) / total_groups + 1 : 0;
    const uint32_t last = g < N ? g + (nrows - 1) * total_groups : N - 1;
    const uint32_t pc = min(static_cast<uint32_t>(lane), npairs - 1);
    const uint32_t keep = static_cast<uint32_t>(lane) < npairs ? 0xFFFFFFFFu : 0u;  // NaN-safe drop of idle lanes

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

    // x first: thread t loads 16-byte chunk t (clamped) to xs + 16 t, and
    // every wave's x load is issued before any weight load of the workgroup.
    const uint32_t xc = min(static_cast<uint32_t>(tid), npairs * 8 - 1);
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t*>(x) + 16u * xc,
                                     (lds_ptr)(xs + 1024u * static_cast<uint32_t>(wave)), 16, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // Waits until at most `rows` rows' loads (rows <= D, wave-uniform) are
    // outstanding (vmcnt counts in issue order).
    auto wait_rows = [&](uint32_t rows) {
        if (rows >= 3 && D >= 3) __builtin_amdgcn_s_waitcnt(0x0F70 | (LOADS * 3));
        else if (rows == 2 && D >= 2) __builtin_amdgcn_s_waitcnt(0x0F70 | (LOADS * 2));
        else if (rows == 1) __builtin_amdgcn_s_waitcnt(0x0F70 | LOADS);
        else __builtin_amdgcn_s_waitcnt(0x0F70);
    };
#pragma unroll
    for (int d = 0; d < D; ++d)
        if (static_cast<uint32_t>(d) < nrows) load_row(static_cast<uint32_t>(d), static_cast<uint32_t>(d));
    __builtin_amdgcn_sched_barrier(0);
    // no more than this wave's first rows' loads outstanding means its x
    // chunk has landed; the barrier then covers every wave's
    wait_rows(nrows < static_cast<uint32_t>(D) ? nrows : static_cast<uint32_t>(D));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    XPair xv;
    {
        uint32_t xr[32];
        const uint8_t* slot = xs + pc * 128u;
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
        xv.c0 = (-8.0f / 1048576.0f) * s0;
        xv.c1 = (-8.0f / 1048576.0f) * s1;
        order_x(xr, xv);
    }

    // Row sums stay in lanes (lane j % 64 holds row j) and are stored every 64
    // rows and at the end.
    float mine = 0.0f;
    for (uint32_t j = 0; j < nrows; ++j) {
        // Rows are loaded only up to the wave's last, so the loads left in
        // flight once row j has landed shrink at the end.
        if (j + D < nrows) {
            load_row(j + D, (j + D) % R);
            __builtin_amdgcn_s_waitcnt(0x0F70 | (LOADS * D));
        } else {
            wait_rows(nrows - 1 - j);
        }
        const uint32_t* pr = reinterpret_cast<const uint32_t*>(ring + (j % R) * row_bytes + pc * kPairBytes);
        uint32_t raw[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) raw[i] = pr[i];
        const float part = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, pair_dot(raw, xv)) & keep);
        const float s = wave_sum(part);
        mine = static_cast<uint32_t>(lane) == (j & 63u) ? s : mine;
        if ((j & 63u) == 63u || j + 1 == nrows) {
            const uint32_t first = j & ~63u;
            if (static_cast<uint32_t>(lane) <= (j & 63u))
                y[g + (first + static_cast<uint32_t>(lane)) * total_groups] = to_out<OutT>(1048576.0f * mine);
        }
    }
}

template <int R, int D>
hipError_t launch_gemv_lds(const Problem& p) {
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        return n;
    }();
    const uint32_t row_bytes = p.K / 64 * kPairBytes;
    const uint32_t loads = (row_bytes / 16 + 63) / 64;
    uint32_t groups = static_cast<uint32_t>(cus);
    const uint32_t need = (p.N + kWaves - 1) / kWaves;  // no workgroup without a row
    if (groups > need) groups = need;
    const size_t lds = static_cast<size_t>(kWaves) * R * row_bytes;
    const dim3 grid(groups), block(kThreads);
    const auto* x = static_cast<const uint16_t*>(p.x);
    const auto* w = static_cast<const uint8_t*>(p.w);
    const uint32_t total = groups * kWaves;
#define MOTE_LDS_LAUNCH(L)                                                                                      \
    do {                                                                                                        \
        if (p.out == OutType::F32)                                                                              \
            hipLaunchKernelGGL((gemv_lds_kernel<R, D, L, float>), grid, block, lds, p.stream, x, w,            \
                               static_cast<float*>(p.y), p.N, p.K, total);                                    \
        else                                                                                                    \
            hipLaunchKernelGGL((gemv_lds_kernel<R, D, L, _Float16>), grid, block, lds, p.stream, x, w,         \
                               static_cast<_Float16*>(p.y), p.N, p.K, total);                                 \
    } while (0)
    switch (loads) {
        case 1: MOTE_LDS_LAUNCH(1); break;
        case 2: MOTE_LDS_LAUNCH(2); break;
        case 3: MOTE_LDS_LAUNCH(3); break;
        default: return hipErrorInvalidValue;
    }
#undef MOTE_LDS_LAUNCH
    return hipGetLastError();
}

// p0 = ring slots, p1 = rows in flight.
const Variant kLds[] = {
    Variant{"rowlds_r2d1", Kind::GemvLds, 2, 1, 0, &launch_gemv_lds<2, 1>},
    Variant{"rowlds_r3d1", Kind::GemvLds, 3, 1, 0, &launch_gemv_lds<3, 1>},
    Variant{"rowlds_r3d2", Kind::GemvLds, 3, 2, 0, &launch_gemv_lds<3, 2>},
};

}  // namespace

const Variant* gemv_lds_variants(int* count) {
    *count = static_cast<int>(sizeof(kLds) / sizeof(kLds[0]));
    return kLds;
}

// One token, K a multiple of 256 from 256 to 4096 (rows start on 16-byte
// boundaries), weights and x 16-byte aligned (the direct-to-LDS loads move
// aligned 16-byte chunks).
bool gemv_lds_supports(const Variant& v, const Problem& p) {
    (void)v;
    return p.M == 1 && p.K % 256 == 0 && p.K >= 256 && p.K <= kMaxK && reinterpret_cast<uintptr_t>(p.w) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(p.x) % 16 == 0 && p.w_up == nullptr;
}

}  // namespace mote::q4_0

// Q4_0 skinny GEMM (2 <= M <= 64) on the CDNA4 matrix cores.
//
// Computes y[m, n] = sum_k x[m, k] * w[n, k] for f16 x [M, K] and GGML Q4_0
// w [N, K], the operation of crates/mote-backend-hip/src/
// quantized_linear.hip:13-52 (oracle crates/mote-reference/src/
// quantized.rs:89-144).  With a handful of tokens the vector-ALU dot products
// cost M K N / 2 v_dot2 operations and bound the kernel; here the products run
// on v_mfma_f32_16x16x32_f16 and the vector ALUs only dequantise, so the
// weight stream from HBM stays the bound up to 16 tokens per token tile.
//
// Mapping:
//  * a workgroup is KS waves; wave kw owns the K slice of STEPS x 4 block pairs
//    starting at pair 4 STEPS kw, and keeps the activations of its slice for
//    the workgroup's tokens in registers for the whole kernel;
//  * the workgroups walk (16-row tile, token group) items persistently, a
//    token group being MT 16-token tiles that share each dequantised weight
//    operand (a workgroup keeps one token group for the whole kernel); per
//    item and step, lane (i, g) = (lane % 16, lane / 16) loads block pair
//    4 (STEPS kw + s) + g of row i of the tile (36 bytes, the same dword-
//    aligned load as the GEMV), dequantises it in registers to binary16
//    (q - 8) * d (exact q - 8 from the 1024 + q and 64 + q exponent tricks,
//    one rounding of the product), and feeds the 8 MFMAs of the step: MFMA t takes nibble
//    dword t of every lane's pair, so one MFMA spans the same 8 positions of
//    the 4 pairs of its lane groups, and the activation operand holds x at
//    exactly those positions (any consistent order of k is exact for a dot);
//  * the KS partial 16 x 16 tiles meet in LDS and are summed in a fixed order
//    (deterministic), then written as f32 or f16.
//
// The next item's weight loads are issued before the current item's MFMAs.
//
// Q8_0 weights (Q8): a pair is 68 bytes (17 dwords); MFMA t takes elements
// 8t .. 8t + 7 of each lane's pair, dequantised by dequant8_q8 into a binary16
// hi + lo pair (two MFMAs, so the 8-bit products keep 22 bits), and the
// activation operand holds x at those positions in the same order.
//
// Fused gate/up (GU, RT = 2): row tile 0 of an item is rows n .. n + 15 of the
// gate matrix and row tile 1 the same rows of the up matrix, and the store
// writes y[m, n] = silu(gate) * up (the operation the prefill kernels fuse for
// M >= 64).
#include "common.hpp"
#include "q4_0.hpp"
#include "skinny_mfma.hpp"

#include <cstring>
#include <type_traits>

namespace mote::q4_0 {
namespace {

template <typename OutT, bool GU>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, uint32_t kparts,
                                                            uint64_t count, OutT* __restrict__ y) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x; i < count;
         i += static_cast<uint64_t>(gridDim.x) * 256) {
        float s = sum_parts(part, kparts, count, i);
        if constexpr (GU) s = silu(s) * sum_parts(part + static_cast<uint64_t>(kparts) * count, kparts, count, i);
        y[i] = to_out<OutT>(s);
    }
}

template <int KS, int STEPS, int MT, int D, int G, int RT, bool TR = false, int LAZY = 0, bool XC = false,
          bool GU = false, bool Q8 = false, bool XW = false, bool SK = false>
hipError_t launch_skinny(const Problem& p) {
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        return n;
    }();
    const SkinnyGrid sg = skinny_grid<KS, STEPS, MT, G, RT, LAZY, GU, SK>(p.M, p.N, p.K, cus);
    if (!sg.ok) return hipErrorInvalidConfiguration;
    constexpr uint32_t kItemRows = GU ? 16u : 16u * RT;
    const uint32_t row_tiles = (p.N + kItemRows - 1) / kItemRows;
    const uint32_t token_groups = sg.token_groups, kparts = sg.kparts, items = sg.items, groups = sg.groups;
    const uint32_t per_xcd = sg.per_xcd;
    const dim3 grid(groups), block(KS * 64);
    float* part = nullptr;
    uint32_t* counters = nullptr;
    bool fold = false;
    const uint64_t count = static_cast<uint64_t>(p.M) * p.N;
    // Split K: the stream's scratch lock is held until every kernel of the
    // call is queued (the lease goes out of scope at return).
    ScratchPool::Lease lease;
    if constexpr (SK) {
        const size_t need = kSplitKCounterBytes + count * kparts * (GU ? 2 : 1) * sizeof(float);
        uint8_t* base = nullptr;
        if (p.scratch != nullptr) {  // the caller's buffer: too small is an error, before any launch
            if (need > p.scratch_bytes) return hipErrorOutOfMemory;
            base = reinterpret_cast<uint8_t*>(p.scratch);
        } else {
            const hipError_t e = acquire_scratch(p.stream, need, &lease);
            if (e != hipSuccess) return e;
            base = static_cast<uint8_t*>(lease.ptr());
            if (lease.fresh()) {  // a new buffer: its counters start at zero
                const hipError_t z = launch_zero_fill(base, kSplitKCounterBytes / 4, OutType::F32, p.stream);
                if (z != hipSuccess) return z;
            }
        }
        part = reinterpret_cast<float*>(base + kSplitKCounterBytes);
        fold = p.splitk_fold && static_cast<uint64_t>(row_tiles) * token_groups <= kSplitKCounterBytes / 4;
        if (fold) counters = reinterpret_cast<uint32_t*>(base);
    }
    if (p.out == OutType::F32) {
        hipLaunchKernelGGL((skinny_mfma_kernel<KS, STEPS, MT, D, RT, TR, float, LAZY, XC, GU, Q8, XW, SK>), grid,
                           block, 0, p.stream, static_cast<const uint16_t*>(p.x), static_cast<const uint8_t*>(p.w),
                           static_cast<const uint8_t*>(p.w_up), static_cast<float*>(p.y), p.M, p.N, p.K,
                           token_groups, items, per_xcd, part, kparts, counters);
    } else {
        hipLaunchKernelGGL((skinny_mfma_kernel<KS, STEPS, MT, D, RT, TR, _Float16, LAZY, XC, GU, Q8, XW, SK>), grid,
                           block, 0, p.stream, static_cast<const uint16_t*>(p.x), static_cast<const uint8_t*>(p.w),
                           static_cast<const uint8_t*>(p.w_up), static_cast<_Float16*>(p.y), p.M, p.N, p.K,
                           token_groups, items, per_xcd, part, kparts, counters);
    }
    if constexpr (SK) {
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess || fold) return e;
        const uint64_t blocks64 = (count + 255) / 256;
        const dim3 rgrid(static_cast<uint32_t>(blocks64 < 2048 ? blocks64 : 2048)), rblock(256);
        if (p.out == OutType::F32)
            hipLaunchKernelGGL((splitk_reduce_kernel<float, GU>), rgrid, rblock, 0, p.stream, part, kparts, count,
                               static_cast<float*>(p.y));
        else
            hipLaunchKernelGGL((splitk_reduce_kernel<_Float16, GU>), rgrid, rblock, 0, p.stream, part, kparts, count,
                               static_cast<_Float16*>(p.y));
    }
    return hipGetLastError();
}

#define MOTE_SKINNY(KS, STEPS, MT, D, G, RT)                                                     \
    Variant{"skinny_mfma_k" #KS "_s" #STEPS "_t" #MT "_d" #D "_g" #G "_r" #RT, Kind::SkinnyMfma, KS, \
            STEPS, MT, &launch_skinny<KS, STEPS, MT, D, G, RT>}
#define MOTE_SKINNY_TRLC(KS, STEPS, MT, G, L)                                                    \
    Variant{"skinny_mfma_k" #KS "_s" #STEPS "_t" #MT "_d1_g" #G "_r1_tr_l" #L "_c", Kind::SkinnyMfma, \
            KS, STEPS, MT, &launch_skinny<KS, STEPS, MT, 1, G, 1, true, L, true>}
#define MOTE_SKINNY_GU(KS, STEPS, MT, D, L, XC, SUFFIX)                                           \
    Variant{"gateup_skinny_k" #KS "_s" #STEPS "_t" #MT "_d" #D SUFFIX, Kind::GateUpSkinny, KS, STEPS, MT, \
            &launch_skinny<KS, STEPS, MT, D, 1, 2, true, L, XC, true>}
#define MOTE_SKINNY_Q8(KS, STEPS, MT, D, L, XC, SUFFIX)                                          \
    Variant{"q8_skinny_k" #KS "_s" #STEPS "_t" #MT "_d" #D SUFFIX, Kind::Q8Skinny, KS, STEPS, MT,    \
            &launch_skinny<KS, STEPS, MT, D, 1, 1, true, L, XC, false, true>}
// x first (_w): the activations are loaded and converted before the first
// weight load.
#define MOTE_SKINNY_W(KS, STEPS, MT, L, XC, SUFFIX)                                                 \
    Variant{"skinny_mfma_k" #KS "_s" #STEPS "_t" #MT "_d1_g1_r1_tr_l" #L SUFFIX "_w", Kind::SkinnyMfma, KS, \
            STEPS, MT, &launch_skinny<KS, STEPS, MT, 1, 1, 1, true, L, XC, false, false, true>}
#define MOTE_SKINNY_GU_W(KS, STEPS, MT, L, XC, SUFFIX)                                              \
    Variant{"gateup_skinny_k" #KS "_s" #STEPS "_t" #MT "_d1_l" #L SUFFIX "_w", Kind::GateUpSkinny, KS, STEPS, \
            MT, &launch_skinny<KS, STEPS, MT, 1, 1, 2, true, L, XC, true, false, true>}
#define MOTE_SKINNY_Q8_W(KS, STEPS, MT, L, XC, SUFFIX)                                              \
    Variant{"q8_skinny_k" #KS "_s" #STEPS "_t" #MT "_d1_l" #L SUFFIX "_w", Kind::Q8Skinny, KS, STEPS, MT, \
            &launch_skinny<KS, STEPS, MT, 1, 1, 1, true, L, XC, false, true, true>}
// Split K (_sk): K any multiple of KS x STEPS x 256, cut into that many
// parts; partial tiles in a per-stream scratch buffer, added in part order by
// the last workgroup of each tile (or, with the fold off, a second kernel).
#define MOTE_SKINNY_SK(KS, STEPS, MT, L, SUFFIX)                                                   \
    Variant{"skinny_mfma_k" #KS "_s" #STEPS "_t" #MT "_d1_g1_r1_tr_l" #L SUFFIX "_w_sk", Kind::SkinnyMfma, KS, \
            STEPS, MT, &launch_skinny<KS, STEPS, MT, 1, 1, 1, true, L, true, false, false, true, true>}
#define MOTE_SKINNY_Q8_SK(KS, STEPS, MT, L, SUFFIX)                                                \
    Variant{"q8_skinny_k" #KS "_s" #STEPS "_t" #MT "_d1_l" #L SUFFIX "_w_sk", Kind::Q8Skinny, KS, STEPS, MT, \
            &launch_skinny<KS, STEPS, MT, 1, 1, 1, true, L, true, false, true, true, true>}
#define MOTE_SKINNY_GU_SK(KS, STEPS, MT, L, SUFFIX)                                                \
    Variant{"gateup_skinny_k" #KS "_s" #STEPS "_t" #MT "_d1_l" #L SUFFIX "_w_sk", Kind::GateUpSkinny, KS, STEPS, \
            MT, &launch_skinny<KS, STEPS, MT, 1, 1, 2, true, L, true, true, false, true, true>}
#define MOTE_SKINNY_TR(KS, STEPS, MT, D, G)                                                       \
    Variant{"skinny_mfma_k" #KS "_s" #STEPS "_t" #MT "_d" #D "_g" #G "_r1_tr", Kind::SkinnyMfma, KS, \
            STEPS, MT, &launch_skinny<KS, STEPS, MT, D, G, 1, true>}

// The tiles the dispatch heuristic picks, the one-slice fallbacks for K =
// 1024 and 2048, and three measured alternatives (one item per barrier, and
// the deferred reduction with the weight loads issued before the
// activations).
const Variant kSkinny[] = {
    MOTE_SKINNY(8, 1, 1, 1, 1, 1), MOTE_SKINNY(4, 1, 1, 1, 1, 1),
    MOTE_SKINNY_TR(8, 2, 1, 1, 1), MOTE_SKINNY_TRLC(16, 1, 1, 1, 4), MOTE_SKINNY_TRLC(8, 2, 1, 1, 8),
    MOTE_SKINNY_W(16, 1, 1, 4, true, "_c"), MOTE_SKINNY_W(8, 2, 1, 8, true, "_c"),
    MOTE_SKINNY_W(8, 2, 2, 4, true, "_c"), MOTE_SKINNY_W(8, 2, 2, 8, true, "_c"),
    MOTE_SKINNY_GU(8, 2, 1, 1, 0, false, ""), MOTE_SKINNY_GU(8, 2, 2, 1, 0, true, "_c"),
    MOTE_SKINNY_GU_W(16, 1, 1, 4, false, ""), MOTE_SKINNY_GU_W(16, 1, 1, 4, true, "_c"),
    MOTE_SKINNY_GU_W(8, 2, 1, 8, true, "_c"), MOTE_SKINNY_GU_W(8, 2, 2, 4, true, "_c"),
    MOTE_SKINNY_Q8(16, 1, 2, 1, 0, true, "_c"),
    MOTE_SKINNY_Q8_W(16, 1, 1, 4, false, ""), MOTE_SKINNY_Q8_W(16, 1, 1, 4, true, "_c"),
    MOTE_SKINNY_Q8_W(8, 2, 1, 8, true, "_c"), MOTE_SKINNY_Q8_W(8, 2, 2, 4, true, "_c"),
    // split K, parts of 2048 or 4096
    MOTE_SKINNY_SK(8, 1, 1, 4, "_c"), MOTE_SKINNY_SK(8, 1, 1, 8, "_c"), MOTE_SKINNY_SK(8, 1, 2, 4, "_c"),
    MOTE_SKINNY_SK(8, 1, 2, 8, "_c"), MOTE_SKINNY_SK(16, 1, 1, 4, "_c"), MOTE_SKINNY_SK(8, 2, 1, 8, "_c"),
    MOTE_SKINNY_SK(8, 2, 2, 8, "_c"),
    MOTE_SKINNY_Q8_SK(8, 1, 1, 4, "_c"), MOTE_SKINNY_Q8_SK(8, 1, 1, 8, "_c"), MOTE_SKINNY_Q8_SK(8, 1, 2, 8, "_c"),
    MOTE_SKINNY_GU_SK(8, 1, 1, 4, "_c"), MOTE_SKINNY_GU_SK(8, 1, 1, 8, "_c"), MOTE_SKINNY_GU_SK(8, 1, 2, 8, "_c"),
    // parts of 1024 for K a multiple of 1024 only (2048 for the gate/up)
    MOTE_SKINNY_SK(4, 1, 1, 8, "_c"), MOTE_SKINNY_SK(4, 1, 2, 8, "_c"), MOTE_SKINNY_GU_SK(4, 1, 1, 8, "_c"),
    MOTE_SKINNY_GU_SK(4, 1, 2, 8, "_c"), MOTE_SKINNY_Q8_SK(4, 1, 1, 8, "_c"), MOTE_SKINNY_Q8_SK(4, 1, 2, 8, "_c"),
};

#undef MOTE_SKINNY
#undef MOTE_SKINNY_TR
#undef MOTE_SKINNY_TRLC
#undef MOTE_SKINNY_GU
#undef MOTE_SKINNY_Q8
#undef MOTE_SKINNY_W
#undef MOTE_SKINNY_SK
#undef MOTE_SKINNY_Q8_SK
#undef MOTE_SKINNY_GU_SK
#undef MOTE_SKINNY_GU_W
#undef MOTE_SKINNY_Q8_W

}  // namespace

const Variant* skinny_mfma_variants(int* count) {
    *count = static_cast<int>(sizeof(kSkinny) / sizeof(kSkinny[0]));
    return kSkinny;
}

// K exactly KS * STEPS * 256 (each wave one K slice of whole steps), x 16-byte
// and w (and the up matrix of a gate/up) dword aligned, at most 64 tokens (MT
// token tiles per pass, RT row tiles per item).
bool skinny_mfma_supports(const Variant& v, const Problem& p) {
    const uint32_t span = static_cast<uint32_t>(v.p0) * static_cast<uint32_t>(v.p1) * 256u;
    const size_t len = std::strlen(v.name);
    if (len > 3 && std::strcmp(v.name + len - 3, "_sk") == 0) {  // split K: any multiple of the slice, two parts or more
        const bool up_ok = v.kind == Kind::GateUpSkinny
                               ? p.w_up != nullptr && reinterpret_cast<uintptr_t>(p.w_up) % 4 == 0
                               : p.w_up == nullptr;
        return p.M >= 1 && p.M <= 64 && p.K >= 2 * span && p.K % span == 0 && reinterpret_cast<uintptr_t>(p.w) % 4 == 0 &&
               reinterpret_cast<uintptr_t>(p.x) % 16 == 0 && up_ok;
    }
    const bool up_ok = v.kind != Kind::GateUpSkinny ||
                       (p.w_up != nullptr && reinterpret_cast<uintptr_t>(p.w_up) % 4 == 0);
    return p.M >= 1 && p.M <= 64 && p.K == span && reinterpret_cast<uintptr_t>(p.w) % 4 == 0 &&
           reinterpret_cast<uintptr_t>(p.x) % 16 == 0 && up_ok;
}

}  // namespace mote::q4_0

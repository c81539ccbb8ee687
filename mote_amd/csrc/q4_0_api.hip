// C ABI of the Q4_0 quantized-linear path and its per-(M, N, K) dispatch cache.
//
// mote_hip_quantized_linear_q4_0_f16 keeps the signature, argument meaning and
// status codes of crates/mote-backend-hip/src/quantized_linear.hip:56-91:
// null pointers or K % 32 != 0 -> hipErrorInvalidValue (1); rows == 0 or N == 0
// -> 0 without a launch; rows * N > UINT_MAX -> hipErrorInvalidConfiguration
// (9); K == 0 launches and writes zeros; otherwise the launch status.
//
// The dispatch context mirrors the plan cache of the reference's hipBLASLt
// shim (crates/mote-backend-hip/src/hipblaslt_shim.cpp:43-46, 156-249,
// 352-408): one mutex-guarded map per handle from the problem key to the
// chosen kernel variant; on a miss the variant is either picked by the shape
// heuristic or, with autotuning on, by timing every eligible variant with
// hipEvents on the caller's stream (each candidate writes the caller's output,
// which the final launch overwrites).  Later calls only launch.
#include <hip/hip_runtime.h>

#include "export.hpp"

#include <algorithm>
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "q4_0.hpp"

namespace mote::q4_0 {
namespace {

enum class Op : int { Linear = 0, GateUp = 1, LinearQ8 = 2 };

struct Key {
    uint32_t m, n, k;
    int op, out, align;  // align: align_class() of the operands
    bool operator<(const Key& o) const {
        return std::tie(m, n, k, op, out, align) < std::tie(o.m, o.n, o.k, o.op, o.out, o.align);
    }
};

struct Dispatcher {
    std::mutex mutex;
    std::map<Key, const Variant*> plans;
    bool autotune = false;
    bool splitk_fold = false;
    std::string forced;
    std::string last_error;
};

std::vector<const Variant*> all_variants() {
    std::vector<const Variant*> out;
    int count = 0;
    for (auto table : {gemv_lds_variants, gemv_stream_variants, gemv_rows_variants, gemv_variants,
                       skinny_mfma_variants, prefill_variants, generic_variants}) {
        const Variant* v = table(&count);
        for (int i = 0; i < count; ++i) out.push_back(&v[i]);
    }
    return out;
}

const Variant* find_variant(const std::string& name) {
    for (const Variant* v : all_variants())
        if (name == v->name) return v;
    return nullptr;
}

bool kind_matches(const Variant& v, Op op) {
    if (op == Op::GateUp)
        return v.kind == Kind::GateUpMfma || v.kind == Kind::GateUpSkinny || v.kind == Kind::GateUpStream ||
               v.kind == Kind::GateUpGeneric;
    if (op == Op::LinearQ8)
        return v.kind == Kind::Q8Stream || v.kind == Kind::Q8Lds || v.kind == Kind::Q8Skinny ||
               v.kind == Kind::Q8Prefill || v.kind == Kind::Q8Generic;
    return v.kind == Kind::Gemv || v.kind == Kind::GemvRows || v.kind == Kind::GemvStream ||
           v.kind == Kind::GemvLds || v.kind == Kind::SkinnyMfma || v.kind == Kind::Mfma || v.kind == Kind::Generic;
}

bool supports(const Variant& v, const Problem& p) {
    switch (v.kind) {
        case Kind::Gemv: return gemv_supports(v, p);
        case Kind::GemvRows: return gemv_rows_supports(v, p);
        case Kind::GemvLds:
        case Kind::Q8Lds: return gemv_lds_supports(v, p);
        case Kind::GemvStream:
        case Kind::GateUpStream:
        case Kind::Q8Stream: return gemv_stream_supports(v, p);
        case Kind::SkinnyMfma:
        case Kind::GateUpSkinny:
        case Kind::Q8Skinny: return skinny_mfma_supports(v, p);
        case Kind::Mfma:
        case Kind::GateUpMfma:
        case Kind::Q8Prefill: return prefill_supports(v, p);
        default: return true;
    }
}

bool fast_eligible(const Problem& p) {
    return p.K % 64 == 0 && reinterpret_cast<uintptr_t>(p.w) % 4 == 0 &&
           reinterpret_cast<uintptr_t>(p.x) % 16 == 0 &&
           (p.w_up == nullptr || reinterpret_cast<uintptr_t>(p.w_up) % 4 == 0);
}

// The operands' alignment class, part of the plan key: 0 when only the
// generic kernels run (K % 64 != 0, or weights off the 4-byte grid), 1 when
// the kernels with dword weight loads run, 2 when the weights (both matrices
// of a gate/up) and the activations also sit on the 16-byte grid that the
// direct-to-LDS ring kernels load in 16-byte chunks.  A plan made for one
// class is never reused for another.
int align_class(const Problem& p) {
    if (!fast_eligible(p)) return 0;
    const bool a16 = reinterpret_cast<uintptr_t>(p.w) % 16 == 0 && reinterpret_cast<uintptr_t>(p.x) % 16 == 0 &&
                     (p.w_up == nullptr || reinterpret_cast<uintptr_t>(p.w_up) % 16 == 0);
    return a16 ? 2 : 1;
}

// Variants the autotuner may time: the matrix-core kernels only for M >= 64
// (prefill shapes), the vector-ALU kernels below that.
std::vector<const Variant*> candidates(const Problem& p, Op op) {
    std::vector<const Variant*> out;
    for (const Variant* v : all_variants()) {
        if (!kind_matches(*v, op) || !supports(*v, p)) continue;
        const bool generic = v->kind == Kind::Generic || v->kind == Kind::GateUpGeneric;
        if (generic && fast_eligible(p)) continue;
        const bool vector_alu = v->kind == Kind::Gemv || v->kind == Kind::GemvRows || v->kind == Kind::GemvLds ||
                                v->kind == Kind::GemvStream || v->kind == Kind::Q8Stream ||
                                v->kind == Kind::GateUpStream || v->kind == Kind::Q8Lds;
        if (vector_alu && p.M >= 64) continue;
        const bool skinny = v->kind == Kind::SkinnyMfma || v->kind == Kind::GateUpSkinny || v->kind == Kind::Q8Skinny;
        if (skinny && p.M > 64) continue;
        if ((v->kind == Kind::Mfma || v->kind == Kind::GateUpMfma || v->kind == Kind::Q8Prefill) && p.M < 64)
            continue;
        out.push_back(v);
    }
    return out;
}

int device_cus() {
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        return n;
    }();
    return cus;
}

const Variant* by_name(const char* name) {
    const Variant* v = find_variant(name);
    return v;
}

// Output tiles of a BM x BN prefill tiling of the problem.
uint64_t prefill_tiles(const Problem& p, uint32_t bm, uint32_t bn) {
    return static_cast<uint64_t>((p.M + bm - 1) / bm) * ((p.N + bn - 1) / bn);
}

// The tile `base` with the most block pairs per step (barrier) up to max_kp
// that K allows (`<base>_k<kp>`), else `base` itself.  More k per step
// amortises the step's barrier and operand ramp: measured on MI355X at K =
// 4096, N = 14 336, 128 x 256 with 2 pairs 69.7 us against 73.5 at 512
// tokens, 128 x 128 with 2 pairs 45.0 against 47.4 at 256, 64 x 128 with 4
// pairs 26.0-27.4 against 38.8 at 128 (gate/up 130.6 against 137.6 us at 512
// tokens, 88.3 against 117.8 us at 64 x 8192 x 28 672).
const Variant* deepest_step(const char* base, const Problem& p, int max_kp) {
    char name[80];
    for (int kp = max_kp; kp >= 2; kp /= 2) {
        std::snprintf(name, sizeof name, "%s_k%d", base, kp);
        const Variant* v = by_name(name);
        if (v && prefill_supports(*v, p)) return v;
    }
    return by_name(base);
}

// A prefill tile: the variant family, the deepest step to try, and the
// measured time of one dispatch wave of such tiles (one per CU) at K = 4096.
struct TileCost {
    const char* base;
    int max_kp;
    float wave_us;
};

// The tile minimising the modelled time, dispatch waves (ceil(tiles / CUs):
// a partial last wave costs a whole one) times the wave time; ties go to the
// earlier (larger) tile.  Null when K allows none of them a multi-pair step.  Measured on MI355X, the model picks the fastest
// tile at every shape timed (64-1024 tokens, N = 4096-14 336, K = 4096 and
// 14 336); e.g. 256 x 4096 x 4096 on 64 x 64 tiles in 18.9 us (the rule
// "first tile with >= 200 tiles" fell to the 16 x 16 tiles: 39.5 us), 384 x
// 4096 x 14 336 on 128 x 256 tiles in 59.4 us (128 x 128: 80.4 us).
template <int N>
const Variant* cheapest_tiles(const Problem& p, const TileCost (&cand)[N]) {
    const uint64_t cus = static_cast<uint64_t>(device_cus());
    const Variant* best = nullptr;
    float best_us = 0.0f;
    for (const TileCost& c : cand) {
        const Variant* v = deepest_step(c.base, p, c.max_kp);
        // the wave times hold for multi-pair steps; where K allows only one
        // pair per step the caller's rule decides (the 16 x 16 tiles measure
        // as fast there: Q8_0 128 x 4160 x 14 336 62.5 us against 64.5)
        if (!v || v == by_name(c.base) || !prefill_supports(*v, p)) continue;
        const uint64_t waves = (prefill_tiles(p, static_cast<uint32_t>(v->p0), static_cast<uint32_t>(v->p1)) + cus - 1) / cus;
        const float us = static_cast<float>(waves) * c.wave_us;
        if (!best || us < best_us) {
            best = v;
            best_us = us;
        }
    }
    return best;
}

// The Q8_0 linear's prefill tiles and their wave times at K = 4096.
const TileCost kQ8Tiles[] = {{"q8_mfma_x32s_m128_n256_w1", 2, 96.0f},
                             {"q8_mfma_x32s_m128_n128_w1", 2, 56.0f},
                             {"q8_mfma_x32s_m64_n128_w1", 4, 36.0f}};

// The Q4_0 linear's prefill tiles and their wave times at K = 4096.
const TileCost kTiles[] = {{"mfma_x32s_m128_n256_w1", 2, 60.0f},
                           {"mfma_x32s_m128_n128_w1", 2, 40.0f},
                           {"mfma_x32s_m64_n128_w1", 4, 25.0f},
                           {"mfma_x32s_m64_n64_w2", 4, 18.0f}};

// Skinny GEMM (3 <= M <= 64, K = 4096) on the matrix cores, transposed weight
// loads; null when the K slicing does not fit.  One (16-row, token-group) item
// per step of a workgroup, with the reduction deferred over up to 4 items (16
// waves, one K step each) or 8 items (8 waves, two steps); above 4 tokens the
// activations are loaded whole lines per instruction and redistributed through
// LDS (16 x 4096 x 14336: 11.8 us against 12.3 us); with at most one item per
// workgroup 8 waves of two steps without the deferred reduction are fastest
// (4 x 4096 x 4096: 5.7 us against 6.1 us).
//
// Tiles, 3 to 64 tokens: items of one 16-token tile up to 16 tokens or
// while a workgroup owns at most 4 of them, else of two (a 32-token group
// sharing each dequantised weight operand; its 256 KB of activations per CU
// cost more than they save when a workgroup owns one or two items: 32 x 4096
// x 4096 took 9.4 us against 8.4 us).  The activations are loaded and converted before the first weight
// load (_w).  Measured on MI355X at K = 4096, N = 14336 (graph replays,
// weights rotated past the MALL): 4 tokens 9.5 us, 8: 9.5 us, 16: 11.0 us,
// 32: 14.6 us, 64: 20.4 us (the same tiles with the weight loads issued
// first: 9.9, 10.7, 11.9, 15.7 (16-token items) and 21.5 us).
const Variant* skinny_heuristic(const Problem& p) {
    const uint64_t cus = static_cast<uint64_t>(device_cus());
    const uint64_t row_tiles = (p.N + 15) / 16;
    const uint64_t per16 = (row_tiles * ((p.M + 15) / 16) + cus - 1) / cus;  // items per workgroup
    const uint64_t per32 = (row_tiles * ((p.M + 31) / 32) + cus - 1) / cus;
    const char* name;
    // (A one-item 8-wave tile for <= 4 tokens and <= 1 item per CU measured
    // 2-3 % slower than the 16-wave tile below: 3 / 4 x 4096 x 4096 in 5.70 /
    // 5.81 us against 5.57 / 5.65 us.)
    // (Three 16-token tiles at three or more items per workgroup run the
    // 32-token items instead: 36 / 48 x 4096 x 4096 in 9.9 us against 12.7 /
    // 14.3 us; with two items per workgroup the 16-token tiles stay ahead,
    // 48 x 4096 x 2048 in 6.8 against 8.6 us.)
    if (per16 <= 4 && !((p.M + 15) / 16 == 3 && per16 >= 3))
        name = "skinny_mfma_k16_s1_t1_d1_g1_r1_tr_l4_c_w";
    else if (p.M <= 16)
        name = "skinny_mfma_k8_s2_t1_d1_g1_r1_tr_l8_c_w";
    else
        name = per32 <= 4 ? "skinny_mfma_k8_s2_t2_d1_g1_r1_tr_l4_c_w" : "skinny_mfma_k8_s2_t2_d1_g1_r1_tr_l8_c_w";
    const Variant* v = by_name(name);
    return v && skinny_mfma_supports(*v, p) ? v : nullptr;
}

// The fused gate/up up to 64 tokens as a skinny GEMM whose items are one gate
// and one up row tile.  Measured on MI355X at K = 4096, N = 14336: 18.2 us for
// 4 tokens, 19.9 us for 16, 24.4 us for 32 (32-token items, activations
// first) and 35.6 us for 64 (the prefill tiles: 53.0 us); with at most one
// item per workgroup the per-item kernel (8 x 4096 x 4096: 8.5 against 9.6 us).
const Variant* skinny_gate_up_heuristic(const Problem& p) {
    const uint64_t cus = static_cast<uint64_t>(device_cus());
    const uint64_t per16 = ((p.N + 15) / 16 * ((p.M + 15) / 16) + cus - 1) / cus;
    const uint64_t per32 = ((p.N + 15) / 16 * ((p.M + 31) / 32) + cus - 1) / cus;
    const char* name;
    if (p.M <= 16 && per16 <= 1)
        name = "gateup_skinny_k8_s2_t1_d1";
    else if (p.M <= 32 && per16 <= 4)
        name = p.M <= 8 ? "gateup_skinny_k16_s1_t1_d1_l4_w" : "gateup_skinny_k16_s1_t1_d1_l4_c_w";
    else if (p.M <= 16)
        name = "gateup_skinny_k8_s2_t1_d1_l8_c_w";
    else if (p.M <= 32)
        name = "gateup_skinny_k8_s2_t2_d1_l4_c_w";
    else  // up to 4 items per workgroup the lazy 32-token tile (48 x 4096 x 4096: 14.2 against 15.4 us)
        name = per32 <= 4 ? "gateup_skinny_k8_s2_t2_d1_l4_c_w" : "gateup_skinny_k8_s2_t2_d1_c";
    const Variant* v = by_name(name);
    return v && skinny_mfma_supports(*v, p) ? v : nullptr;
}

// Q8_0 skinny GEMM (the Q4_0 kernels' shapes with 68-byte pairs), 3 to 64
// tokens.  Measured on MI355X at K = 4096, N = 14336: 15.5 us at 8 tokens,
// 17.1 us at 16, 21.3 us at 32 (32-token items, activations first) and
// 29.1 us at 64, where the generic kernel took 117-895 us.  (1, 2 and 4
// tokens stay on the streaming GEMV: 4 x 4096 x 4096 in 6.9 us against 8.1
// us here.)
const Variant* skinny_q8_heuristic(const Problem& p) {
    const uint64_t cus = static_cast<uint64_t>(device_cus());
    const uint64_t per16 = ((p.N + 15) / 16 * ((p.M + 15) / 16) + cus - 1) / cus;
    const uint64_t per32 = ((p.N + 15) / 16 * ((p.M + 31) / 32) + cus - 1) / cus;
    const char* name;
    if (p.M <= 32 && per16 <= 4)
        name = p.M <= 8 ? "q8_skinny_k16_s1_t1_d1_l4_w" : "q8_skinny_k16_s1_t1_d1_l4_c_w";
    else if (p.M <= 16)
        name = "q8_skinny_k8_s2_t1_d1_l8_c_w";
    else if (p.M <= 32 || per32 <= 4)  // 48 x 4096 x 4096: 12.5 against 13.1 us on the one below
        name = "q8_skinny_k8_s2_t2_d1_l4_c_w";
    else
        name = "q8_skinny_k16_s1_t2_d1_c";
    const Variant* v = by_name(name);
    return v && skinny_mfma_supports(*v, p) ? v : nullptr;
}

// Split-K skinny GEMM (1 to 64 tokens, K a multiple of 2048 from 8192 up, or
// any K no plain slicing fits): K cut into parts of 2048 or 4096, partial
// tiles added by a second kernel.  Measured on MI355X (the choices below):
//   K = 14336, N = 4096: 2-16 tokens 13.0-14.2 us, 24: 18.9 us, 32: 19.9 us,
//     64: 27.4 us (the vector-ALU GEMV it replaces: 14.9 us at 2 tokens,
//     42.3 at 8, 76.2 at 16, 129.8 at 32);
//   K = 28672, N = 8192: 16 tokens 35.0 us, 32: 45.4 us, 64: 85.6 us;
//   K = 8192, N = 8192: 3 tokens 12.2 us, 16: 13.4 us, 32: 17.5 us, 64:
//     24.5 us (one 8192 slice at 16 tokens: 19.5 us);
//   gate/up K = 8192, N = 28672: 4 tokens 66.0 us, 16: 72.1 us, 32: 92.8 us
//     (the 64 x 128 prefill tiles: 116.6 us at 32 tokens, 117.8 at 48).
// 16-wave workgroups (one per CU) take 4 items while that fits one round of
// CUs; past that, and for 32-token items, 8 items per workgroup of 8 waves
// with the larger K part once the smaller one gives more than 256 workgroups.
const Variant* split_k_heuristic(const Problem& p, Op op) {
    if (p.M > 64 || p.K % 1024 != 0 || p.K < 2048) return nullptr;
    if (p.K % 2048 != 0 || p.K < 4096) {
        // Parts of 1024 (4 waves of 256): K = 3072, 5120, 7168, ... and the
        // gate/up at K = 2048, which no plain slicing fits (a linear at K =
        // 2048 takes the one-slice tiles).
        if (op == Op::Linear && p.K == 2048) return nullptr;
        // 16-token items (measured on MI355X: 32 x 3072 x 8192 in 14.6 us
        // against 21.3 us with 32-token items, 48 / 64 x 5120 x 5120 in 18.0
        // / 22.2 against 24.8 / 26.0; 4 x 5120 x 5120 in 10.9 us against 15.5
        // us on the vector-ALU GEMV); the gate/up takes 32-token items above
        // 32 tokens, and above 16 where the 16-token items exceed 4096 (32 x
        // 5120 x 13824: 48.6 us against 55.5; 32 x 5120 x 5120, 3200 items:
        // 24.1 us against 27.4; 48 / 64 x 5120 x 5120: 32.0 / 33.2 us, where
        // the 16 x 16 prefill tiles took 68.6; 32 x 2048 x 8192: 14.0 against 16.0)
        const uint64_t items1k = static_cast<uint64_t>((p.N + 15) / 16) * ((p.M + 15) / 16) * (p.K / 1024);
        const bool t2 = op == Op::GateUp && (p.M > 32 || (p.M > 16 && (items1k > 4096 || p.K == 2048)));
        const char* name = op == Op::LinearQ8 ? (t2 ? "q8_skinny_k4_s1_t2_d1_l8_c_w_sk" : "q8_skinny_k4_s1_t1_d1_l8_c_w_sk")
                           : op == Op::GateUp ? (t2 ? "gateup_skinny_k4_s1_t2_d1_l8_c_w_sk" : "gateup_skinny_k4_s1_t1_d1_l8_c_w_sk")
                                              : (t2 ? "skinny_mfma_k4_s1_t2_d1_g1_r1_tr_l8_c_w_sk"
                                                    : "skinny_mfma_k4_s1_t1_d1_g1_r1_tr_l8_c_w_sk");
        const Variant* v = by_name(name);
        return v && skinny_mfma_supports(*v, p) ? v : nullptr;
    }
    const uint64_t cus = static_cast<uint64_t>(device_cus());
    const uint64_t row_tiles = (p.N + 15) / 16;
    const uint64_t items2k = row_tiles * ((p.M + 15) / 16) * (p.K / 2048);  // 16-token items, parts of 2048
    const uint64_t items4k = row_tiles * ((p.M + 15) / 16) * (p.K / 4096);
    const uint64_t items2k_t2 = row_tiles * ((p.M + 31) / 32) * (p.K / 2048);  // 32-token items
    const bool k4 = p.K % 4096 == 0;
    const char* name;
    if (op == Op::LinearQ8) {
        // Measured on MI355X: where K is a multiple of 4096, parts of 2048
        // with 8 items per workgroup, 32-token items above 16 tokens (24 /
        // 32 x 8192 x 28672: 71.0 / 75.7 us against 91.1 / 93.4 with 16-token
        // items); otherwise parts of 1024 up to 16 tokens (4 / 16 x 14336 x
        // 4096: 17.7 / 18.6 us against 18.4 / 19.8 with parts of 2048) and
        // parts of 2048 with 8 items per workgroup above (24 / 32 x 14336 x
        // 4096: 27.2 / 28.2 us against 30.1 / 31.0 with 4)
        if (p.M > 32)
            name = "q8_skinny_k8_s1_t2_d1_l8_c_w_sk";
        else if (k4)
            name = p.M > 16 ? "q8_skinny_k8_s1_t2_d1_l8_c_w_sk" : "q8_skinny_k8_s1_t1_d1_l8_c_w_sk";
        else if (p.M > 16)
            name = "q8_skinny_k8_s1_t1_d1_l8_c_w_sk";
        else {
            const Variant* v = by_name("q8_skinny_k4_s1_t1_d1_l8_c_w_sk");
            if (v && skinny_mfma_supports(*v, p)) return v;
            name = "q8_skinny_k8_s1_t1_d1_l4_c_w_sk";
        }
    } else if (op == Op::GateUp) {
        if (p.M > 32) return nullptr;  // the prefill tiles
        if (p.M > 16)
            name = "gateup_skinny_k8_s1_t2_d1_l8_c_w_sk";
        else
            name = items2k > 4 * 512 ? "gateup_skinny_k8_s1_t1_d1_l8_c_w_sk" : "gateup_skinny_k8_s1_t1_d1_l4_c_w_sk";
    } else if (p.M > 16) {
        // where K is a multiple of 4096, by 32-token items of 2048 (measured
        // on MI355X at K = 8192: N = 2048, 32 tokens, 512 items, 16-token
        // items with 4 per workgroup in 9.3 us against 10.8 with 32-token
        // items and 8; 48 / 64 tokens, 1024 items, 4 per workgroup; N = 3072,
        // 48 / 64 tokens, 1536 items, 13.7 / 14.5 us with 8 against 15.3 /
        // 15.4 for the 2-step items)
        // (other K: 16-token items at 33-48 tokens and past 4096 rows, 32 / 48 x
        // 14336 x 5120 in 21.8 / 28.7 us against 24.7 / 36.6, 48 x 14336 x
        // 3584 21.6 against 25.6)
        if (!k4 && (p.M > 32 ? p.M <= 48 : p.N > 4096))
            name = "skinny_mfma_k8_s1_t1_d1_g1_r1_tr_l4_c_w_sk";
        else if (!k4)
            name = p.M > 32 ? "skinny_mfma_k8_s1_t2_d1_g1_r1_tr_l8_c_w_sk" : "skinny_mfma_k8_s1_t2_d1_g1_r1_tr_l4_c_w_sk";
        else if (p.M <= 32 && items2k_t2 <= 512)
            name = "skinny_mfma_k8_s1_t1_d1_g1_r1_tr_l4_c_w_sk";
        else if (items2k_t2 <= 1024)
            name = "skinny_mfma_k8_s1_t2_d1_g1_r1_tr_l4_c_w_sk";
        else if (items2k_t2 <= 8 * 256 && (p.M <= 32 || items2k_t2 < 2048))
            name = "skinny_mfma_k8_s1_t2_d1_g1_r1_tr_l8_c_w_sk";
        else
            name = "skinny_mfma_k8_s2_t2_d1_g1_r1_tr_l8_c_w_sk";
    } else if (k4) {
        // parts of 4096 from two items per CU, parts of 2048 below (4 / 8 / 16
        // x 8192 x 3072, 384 items of 4096: 7.7 / 7.6 / 8.4 us against 8.2 /
        // 8.4 / 9.0; 4 x 8192 x 8192, 1024 items: 12.2 against 12.5)
        name = items4k > 4 * cus   ? "skinny_mfma_k8_s2_t1_d1_g1_r1_tr_l8_c_w_sk"
               : items4k >= 2 * cus ? "skinny_mfma_k16_s1_t1_d1_g1_r1_tr_l4_c_w_sk"
               : items2k > 4 * 512  ? "skinny_mfma_k8_s1_t1_d1_g1_r1_tr_l8_c_w_sk"
                                    : "skinny_mfma_k8_s1_t1_d1_g1_r1_tr_l4_c_w_sk";
    } else {
        // 4 items per workgroup up to 4096 items (4 / 16 x 14336 x 5120, 2240
        // items: 13.9 / 15.8 us against 18.6 / 20.2 with 8)
        name = items2k > 8 * 512 ? "skinny_mfma_k8_s1_t1_d1_g1_r1_tr_l8_c_w_sk"
                                 : "skinny_mfma_k8_s1_t1_d1_g1_r1_tr_l4_c_w_sk";
    }
    const Variant* v = by_name(name);
    return v && skinny_mfma_supports(*v, p) ? v : nullptr;
}

bool splits_k(const Variant& v) {
    const size_t n = std::strlen(v.name);
    return n > 3 && std::strcmp(v.name + n - 3, "_sk") == 0;
}

const Variant* split_k(const Problem& p, Op op, bool split_ok) {
    return split_ok ? split_k_heuristic(p, op) : nullptr;
}

// Rule-based shape heuristic: every shape the plan table does not list.
// split_ok false leaves out the split-K tiles (which need scratch): the
// choice of a call under graph capture whose stream has too little.
const Variant* rules(const Problem& p, Op op, bool split_ok) {
    const bool fast = fast_eligible(p);
    if (op == Op::LinearQ8) {
        // K a multiple of 256: Q8_0 rows through the per-wave LDS ring
        // (q4_0_gemv_lds.hip), one to three tokens per row read up to K =
        // 4096, one token with rows split over S waves above.  Measured on
        // MI355X against the streaming GEMV (or, for three tokens, the skinny
        // tiles): 1 x 4096 x 4096 4.88 us (5.71), x 14336 11.09 (12.46), 2 x
        // 4096 x 14336 12.10 (13.52), 3 x 4096 x 14336 13.17 (14.66), 14336 x
        // 4096 11.41 (12.24), 28672 x 8192 37.95 (41.06).  Four tokens stay
        // on the streaming GEMV (4 x 4096 x 4096: 6.78 us against 8.17).
        if (fast && p.K % 256 == 0 && (p.M <= 3 && p.K <= 4096)) {
            char name[32];
            if (p.M == 1)
                std::snprintf(name, sizeof name, "q8_rowlds_r2d1");
            else
                std::snprintf(name, sizeof name, "q8_rowlds_m%u_r2d1", p.M);
            const Variant* v = by_name(name);
            if (v && gemv_lds_supports(*v, p)) return v;
        }
        if (fast && p.K % 256 == 0 && p.M == 1 && p.K > 4096) {
            uint32_t split = 2;
            while (split < 8 && p.K > 4096u * split) split *= 2;
            char name[32];
            std::snprintf(name, sizeof name, "q8_rowlds_s%u_r2d1", split);
            const Variant* v = by_name(name);
            if (v && gemv_lds_supports(*v, p)) return v;
        }
        // The streaming GEMV over Q8_0 pairs for 1, 2 or 4 tokens (rows split
        // over S waves above K = 4096; one workgroup per CU measured fastest
        // for Q8_0's 68-byte pairs at every Llama shape), the generic kernel
        // otherwise.
        if (fast && (p.M == 1 || p.M == 2 || p.M == 4 || (p.M == 3 && p.K > 4096 && p.K <= 16384))) {
            uint32_t split = 1;
            while (split < 8 && p.K > 4096u * split) split *= 2;
            char name[32];
            // four tokens past K = 4096 where no split-K slicing fits (K %
            // 1024 != 0): rows split over S waves as for two and three
            // (also where split K would take parts of 1024, K % 2048 != 0:
            // 4 x 5120 x 5120 in 10.9 us against 12.7, x 13824 21.1 against
            // 24.8; and at 8192 < K <= 16384 whatever K's slicing: 4 x 14336 x
            // 4096 / 5120 / 6144 in 15.7 / 18.2 / 21.0 us against 17.5 / 24.7 /
            // 27.5 on the split-K tiles)
            const bool m4_split = p.M == 4 && split > 1 && split <= 4 && (p.K % 2048 != 0 || split == 4);
            if (((p.M == 2 || p.M == 3) && split > 1) || m4_split)  // 3 x 8192 x 8192: 15.2 us (split-K tiles 17.6)
                std::snprintf(name, sizeof name, "q8_stream_s%u_m%u_d1q_g1", split, p.M);
            else if (p.M > 1)
                std::snprintf(name, sizeof name, "q8_stream_m%u_d1q_g1", p.M);
            else if (split == 1)
                std::snprintf(name, sizeof name, "q8_stream_d1_g1");
            else
                std::snprintf(name, sizeof name, "q8_stream_s%u_d1_g1", split);
            const Variant* v = by_name(name);
            if (v && gemv_stream_supports(*v, p)) return v;
        }
        if (fast && p.M >= 5 && p.M <= 16 && p.K > 2048 && p.K <= 16384 && p.K % 1024 != 0) {
            // 5-16 tokens where K takes no split-K slicing: passes of up to
            // four tokens on the split-row streaming GEMV (a four-token pass
            // at 11008 x 4096 in 14.9 us; 8 tokens took 76.3 us on the
            // prefill tiles and 89.5 us on the generic kernel; rows split 2
            // ways also below K = 4096: 6 / 8 x 3584 x 4608 in 18.2 / 21.4 us
            // against 27.9 on the prefill tiles)
            char name[40];
            std::snprintf(name, sizeof name, "q8_stream_s%u_m4x_d1q_g1", p.K > 8192 ? 4u : 2u);
            const Variant* v = by_name(name);
            if (v && gemv_stream_supports(*v, p)) return v;
        }
        if (fast && p.M > 32 && p.M <= 64 && p.K > 4096 && prefill_tiles(p, 64, 64) >= 200) {
            // as for Q4_0: 33-64 tokens past K = 4096 on wide rows (48 x 8192
            // x 28672: 81.4 us against 119.3 us on the split-K skinny tiles;
            // 64 x 5120 x 13824: 46.8 against 57.4)
            if (const Variant* v = cheapest_tiles(p, kQ8Tiles)) return v;
        }
        if (fast && p.M <= 64) {
            if (const Variant* v = skinny_q8_heuristic(p)) return v;
            if (const Variant* v = split_k(p, op, split_ok)) return v;
        }
        if (fast && p.M >= 64) {
            // The prefill tiles with 68-byte pairs: the largest 32 x 32 MFMA
            // tile with staging waves that still gives about one tile per CU
            // (measured on MI355X at K = 4096, N = 14336: 256 tokens 67-69 us,
            // 512 tokens 112 us, against 79 and 126 us for 16 x 16 MFMA
            // tiles), the 64 x 64 tiles below (128 tokens: 56.7 us).
            // Each with the deepest step K allows: 2 block pairs per step at
            // 256 tokens 65.0 us (67.8 with one); the 64 x 128 tiles with 4
            // pairs at 128 tokens 40.8 us (61.5 on the 64 x 64 16 x 16 tiles).
            // The tile by dispatch waves and wave time (K = 4096: 128 x 256
            // 96 us, 128 x 128 56 us, 64 x 128 36 us; e.g. 256 x 4096 x 4096
            // in 32.8 us on 64 x 128 tiles against 50.3 on the 16 x 16 tiles,
            // 384 x 4096 x 14 336 in 96.3 us on 128 x 256 against 118.7).
            if (const Variant* v = cheapest_tiles(p, kQ8Tiles)) return v;
            return by_name("q8_mfma_r_m64_n64");
        }
        // tokens with no K slicing (K % 1024 != 0, e.g. 11 008, 13 824): the
        // prefill tiles, where K allows their multi-pair steps
        // (past K = 16384 the generic kernel: 4 / 6 x 18944 x 3584 in 69 /
        // 102 us against 127 us on the tiles)
        if (fast && p.M >= 4 && p.K <= 16384)
            if (const Variant* v = cheapest_tiles(p, kQ8Tiles)) return v;
        return by_name("q8_generic");
    }
    if (op == Op::GateUp) {
        // Up to 64 tokens the skinny gate/up; above, the prefill tiles with
        // raw Q4_0 weights staged in LDS (measured on MI355X at N = 14336,
        // K = 4096: 1.4x-1.8x faster than dequantised f16 weight tiles).
        if (fast && (p.M == 1 || p.M == 2 || (p.M == 3 && p.K > 2048 && p.K <= 16384 && p.K != 4096))) {
            // One or two tokens: the streaming GEMV reading both rows per
            // step (and, for two tokens, each row once for both), rows split
            // over S waves past K = 4096 (measured on MI355X: one token,
            // 4096 x 14336 in 13.6 us, 4.85 TB/s; 8192 x 28672 in 43.9 us,
            // 6.0 TB/s; two tokens, 4096 x 14336 in 15.5 us, 8192 x 28672 in
            // 46.9 us and 14336 x 4096 in 15.0 us, against 17.8, 65.5 and
            // 21.7 us on the skinny tiles; three tokens for 4096 < K <=
            // 16384, rows split up to 4 ways, 8192 x 28672 in 54.4 us against
            // 65.4 us).
            // (three tokens at 2048 < K < 4096 with rows split 2 ways: 3 x
            // 3584 x 18944 in 35.2 us, where the generic kernel took 89.1; 3
            // x 3072 x 8192 16.5 against 18.6 split K)
            uint32_t split = p.M == 3 ? 2 : 1;
            while (split < 8 && p.K > 4096u * split) split *= 2;
            char name[40];
            if (split == 1)
                std::snprintf(name, sizeof name, "%s", p.M == 1 ? "gateup_stream_p1_d1_g1" : "gateup_stream_p1_m2_d1q_g1");
            else
                std::snprintf(name, sizeof name, "gateup_stream_s%u_m%u_d1q_g1", split, p.M);
            const Variant* v = by_name(name);
            if (v && gemv_stream_supports(*v, p)) return v;
        }
        if (fast && p.M > 16 && p.M <= 64 && prefill_tiles(p, 64, 128) >= 200) {
            // 17-64 tokens with at least 200 64 x 128 tiles (wide gate/up,
            // e.g. 28 672 rows): those tiles with 4 block pairs per step beat
            // the split-K skinny tiles (32 x 8192 x 28 672: 91.0 against 96.6
            // us; 48 tokens: 91.8 against 152.0 us)
            const Variant* v = by_name("gateup_mfma_x32s_m64_n128_w1_k4");
            if (v && prefill_supports(*v, p)) return v;
        }
        if (fast && p.M > 32 && p.M <= 64 && prefill_tiles(p, 64, 128) < 200 &&
            (prefill_tiles(p, 64, 64) >= (p.M > 48 ? 160u : 200u) || (p.M > 48 && p.K < 4096))) {
            // 33-64 tokens where 64 x 128 tiles are too few: 64 x 64 tiles of
            // 2 x 2 waves, 4 block pairs per step (64 x 4096 x 14 336: 30.8
            // us, against 35.6 us on the skinny tiles; 64 x 5120 x 13824: 39.9
            // us, where 48 tokens took 71.8 us on the 16 x 16 tiles; 64 x 4096
            // x 11008, 172 tiles: 29.1 us against 31.7 on the skinny tiles;
            // below K = 4096, where the skinny tiles split K in parts of
            // 1024, 64 x 2048 / 3072 x 8192 in 16.5 / 22.4 us against 23.3 /
            // 33.8).  Where the 64 x 64 tiles would take two dispatch waves
            // and the 64 x 128 tiles one, the latter (64 x 3584 x 18944: 40.4
            // us against 53.5)
            const bool two_waves = prefill_tiles(p, 64, 64) > static_cast<uint64_t>(device_cus());
            const Variant* v = two_waves ? deepest_step("gateup_mfma_x32s_m64_n128_w1", p, 4)
                                         : by_name("gateup_mfma_x32s_m64_n64_w2_k4");
            if (v && prefill_supports(*v, p)) return v;
        }
        if (fast && p.M <= 64) {
            if (const Variant* v = skinny_gate_up_heuristic(p)) return v;
            if (const Variant* v = split_k(p, op, split_ok)) return v;
        }
        if (fast && p.M > 32) {
            // 32 x 32 MFMA tiles with staging waves once 128 x 128 tiles give
            // about one per CU (256 tokens: 72.7-75.4 us, 512: 139.5-144.6 us,
            // against 84.5 and 164 us for 16 x 16 tiles); up to 64 tokens
            // the 64 x 128 tiles (64 x 8192 x 28672: 119.4 us, against 150.3
            // us for 128 x 128 tiles); each with the deepest step K allows.
            // (up to 128 tokens where 128 x 128 tiles are too few: 128 x 4096
            // x 14 336 in 45.7 us with 4 pairs per step, against 78.0 us on
            // the 16 x 16 tiles)
            // Above 64 tokens the tile by dispatch waves and wave time (K =
            // 4096: 128 x 128 64 us, 64 x 128 42 us, 64 x 64 30 us; e.g.
            // 256 x 4096 x 4096 in 32.0 us on 64 x 64 tiles against 77.0 on
            // the 16 x 16 tiles, 512 x 4096 x 4096 in 46.7 us on 64 x 128).
            static const TileCost kGateUpTiles[] = {{"gateup_mfma_x32s_m128_n128_w1", 2, 64.0f},
                                                    {"gateup_mfma_x32s_m64_n128_w1", 4, 42.0f},
                                                    {"gateup_mfma_x32s_m64_n64_w2", 4, 30.0f}};
            if (p.M > 64) {
                if (const Variant* v = cheapest_tiles(p, kGateUpTiles)) {
                    // three or more waves of 64 x 128 tiles: 2 block pairs
                    // per step (384 x 4096 x 14 336: 115.4 us against 130.1
                    // with 4; 192 x 8192 x 28 672: 228.1 against 241.9)
                    const Variant* k2 = by_name("gateup_mfma_x32s_m64_n128_w1_k2");
                    const uint64_t waves = (prefill_tiles(p, 64, 128) + device_cus() - 1) / device_cus();
                    if (v == by_name("gateup_mfma_x32s_m64_n128_w1_k4") && waves >= 3 && k2 && prefill_supports(*k2, p))
                        return k2;
                    return v;
                }
            }
            if (p.M <= 128 && prefill_tiles(p, 64, 128) >= 200 && (p.M <= 64 || prefill_tiles(p, 128, 128) < 200))
                return deepest_step("gateup_mfma_x32s_m64_n128_w1", p, 4);
            if (prefill_tiles(p, 128, 128) >= 200) return deepest_step("gateup_mfma_x32s_m128_n128_w1", p, 2);
            return by_name(p.M >= 128 ? "gateup_mfma_r_m128_n64" : "gateup_mfma_r_m64_n64");
        }
        return by_name("gateup_generic");
    }
    if (!fast) return by_name("generic");
    if (p.M > 32 && p.M <= 64 && (p.K > 4096 || p.M == 64) &&
        prefill_tiles(p, 64, 64) >= (p.K > 4096 ? 160u : 200u)) {
        // 33-64 tokens past K = 4096 (64 from K = 4096) with at least 200
        // 64 x 64 tiles (wide rows): the prefill tiles beat the skinny ones
        // (measured on MI355X: 40 / 48 / 64 x 8192 x 28672 on 64 x 128 tiles
        // in 51.8 / 52.3 / 51.3 us against 80.0 / 81.0 / 81.6 us split K; 40
        // x 5120 x 13824 on 64 x 64 tiles in 22.7 us against 31.5; 64 x 4096
        // x 14336 in 17.5 against 18.6; 48 / 64 x 8192 x 10240, 160 tiles,
        // 32.6 / 33.2 us against 35.1 / 39.7).  With fewer tiles (64 x 8192 x
        // 8192, 64 x 14336 x 4096), or 160-199 at K = 4096 (64 x 4096 x
        // 11008: 18.8 against 17.8), the skinny tiles stay ahead.
        if (const Variant* v = cheapest_tiles(p, kTiles)) return v;
    }
    if (p.M > 48 && p.M <= 64 && p.K > 2048 && p.K < 4096) {
        // 49-64 tokens at 2048 < K < 4096, where the skinny tiles split K in
        // parts of 1024 or not at all: the prefill tiles (64 x 3072 x 8192 in
        // 13.6 us against 19.0 on the split-K tiles; 64 x 3072 x 5120 13.5
        // against 14.5)
        if (const Variant* v = cheapest_tiles(p, kTiles)) return v;
    }
    if (p.M == 64) {
        // 64 tokens still run as a skinny GEMM (faster than the prefill tiles).
        const Variant* v = skinny_heuristic(p);
        if (!v) v = split_k(p, op, split_ok);
        if (v) return v;
    }
    if (p.M >= 64) {
        // Prefer the largest tile that still gives about one tile per CU: 32
        // x 32 MFMA tiles with staging waves (measured on MI355X at K = 4096,
        // N = 14336: 128 x 256 at 512 tokens, 68-72 us; 128 x 128 at 256
        // tokens, 46.5-47.1 us; 64 x 128 at 128 tokens, 39.8 us; the 16 x 16
        // tiles took 83, 59.4 and 46.1 us).
        // Each x32s tile with the deepest step K allows (2 block pairs for
        // the 128-row tiles, 4 for 64 x 128 and 64 x 64: what fits the LDS),
        // chosen by dispatch waves and wave time (K = 4096: 128 x 256 60 us,
        // 128 x 128 40 us, 64 x 128 25 us, 64 x 64 18 us).
        if (const Variant* v = cheapest_tiles(p, kTiles)) return v;
        static const char* const order[] = {"mfma_x32s_m128_n256_w1", "mfma_x32s_m128_n128_w1",
                                            "mfma_x32s_m64_n128_w1", "mfma_r_m64_n128", "mfma_r_m64_n64"};
        static const int max_kp[] = {2, 2, 4, 1, 1};
        const Variant* best = nullptr;
        uint64_t best_tiles = 0;
        for (int i = 0; i < 5; ++i) {
            const Variant* v = max_kp[i] > 1 ? deepest_step(order[i], p, max_kp[i]) : by_name(order[i]);
            const uint64_t tiles = static_cast<uint64_t>((p.M + v->p0 - 1) / v->p0) *
                                   ((p.N + v->p1 - 1) / v->p1);
            if (tiles >= 200) return v;
            if (tiles > best_tiles) {
                best = v;
                best_tiles = tiles;
            }
        }
        return best;
    }
    if (p.M == 1) {
        // K a multiple of 256 up to 4096: rows through the per-wave LDS ring
        // with coalesced non-temporal loads (q4_0_gemv_lds.hip), one row in
        // flight beside the one computed (measured on MI355X at K = 4096: N =
        // 14336 7.12-7.27 us, 6144 4.34, 4096 3.73, 1024 3.12, against 7.62,
        // 5.14, 4.22 and 3.51 us for the pair-load GEMV; with x's stage
        // swizzled, two rows in flight measured level or slower at every N:
        // 7.28-7.40, 4.63, 4.17 us, and 5.24 against 5.08 at 8192, 11.82
        // against 11.53 at 28672).
        {
            const Variant* v = by_name("rowlds_r2d1");
            if (v && gemv_lds_supports(*v, p)) return v;
        }
        // K past 4096: rows split over S waves through the LDS ring where
        // each row group owns 8 rows or more and the slices fill 90 % of
        // their load instructions, or 12 rows or more (measured on MI355X:
        // 14336 x 4096 7.90 us, 13824 x 5120 8.90, 5120 x 13824 10.40,
        // 8192 x 28672 22.2, 28672 x 8192 22.2, against 8.04, 9.30, 10.63,
        // 22.6 and 23.8 us for the streaming GEMV below; that one stays ahead
        // at 11008 x 4096, 7.23 us against 7.46, ties at 8192 x 8192, 8.21
        // us, and leads with fewer rows, 14336 x 1024 4.54 us against 4.78).
        if (p.K > 4096 && p.K % 256 == 0) {
            uint32_t s = 2;
            while (s < 8 && p.K > 4096u * s) s *= 2;
            const uint32_t span = (p.K / 64 + s - 1) / s;
            const uint32_t chunks = (span * 36 + 15) / 16, loads = (chunks + 63) / 64;
            const uint64_t rows_per_group = p.N / (static_cast<uint64_t>(device_cus()) * (8u / s));
            const bool full = 10u * chunks >= 9u * 64u * loads;
            if ((rows_per_group >= 8 && full) || rows_per_group >= 12) {
                char name[32];
                std::snprintf(name, sizeof name, "rowlds_s%u_r3d2_g1", s);
                const Variant* v = by_name(name);
                if (v && gemv_lds_supports(*v, p)) return v;
            }
        }
        // Measured on MI355X (graph replays, weights rotated past the MALL):
        // the persistent pipelined GEMV, with rows split over S waves for
        // K > 4096 (4096 x 14336: 7.3 us; 14336 x 4096: 8.0 us, against
        // 9.9 us for the row-streaming GEMV).  Two workgroups per CU pay off
        // once every row group then owns about 1.5 rows or more (4096 x 6144:
        // 5.14 us against 5.35 us; 4096 x 4096: 5.06 us against 4.29 us).
        // The queued form (the next row issued while waiting for the one
        // after the current) wins with one workgroup per CU and with rows
        // split 4 ways (4096 x 4096: 4.18-4.21 us against 4.29-4.30;
        // 14336 x 4096: 7.99-8.06 us against 8.20-8.31), and loses at
        // 8192 x 28672 (23.4 us against 22.5).
        uint32_t split = 1;
        while (split < 8 && p.K > 4096u * split) split *= 2;
        const uint64_t row_groups_g2 = static_cast<uint64_t>(device_cus()) * 2u * (8u / split);
        const unsigned g = 2u * p.N >= 3u * row_groups_g2 ? 2u : 1u;
        char name[32];
        if (split == 1)
            std::snprintf(name, sizeof name, "stream_d1%s_g%u", g == 1 ? "q" : "", g);
        else
            std::snprintf(name, sizeof name, "stream_s%u_d1%s_g%u", split, split == 4 ? "q" : "", g);
        const Variant* st = by_name(name);
        if (st && gemv_stream_supports(*st, p)) return st;
        uint32_t ks = 1;
        while (ks < 8 && p.K > 4096u * ks) ks *= 2;
        std::snprintf(name, sizeof name, "rows_r4_k%u", ks);
        const Variant* rows = by_name(name);
        if (rows && gemv_rows_supports(*rows, p)) return rows;
        if (p.K >= 8192 && p.N <= 8192) return by_name("gemv_r4_t1_k2");
        return by_name(p.N >= 8192 ? "gemv_r4_t1_k1" : "gemv_r2_t1_k1");
    }
    // 2 <= M <= 64: matrix-core skinny GEMM when a K slicing fits (measured on
    // MI355X at K = 4096: 1.2x-7x faster than the vector-ALU dot products from
    // M = 2, and faster than the prefill tiles at M = 64).  One token tile
    // per workgroup up to 16 tokens, double-buffered items above, two token
    // tiles per workgroup above 32 tokens.
    // Two tokens: the vector-ALU streaming GEMV over both tokens at once
    // (4096 x 14336: 9.2 us against 11.9 us on the matrix cores).  From 3
    // tokens: the skinny GEMM of skinny_heuristic, then any skinny variant
    // whose K slicing fits, then the vector-ALU GEMV.
    if (p.K == 4096 && ((p.M == 3 && p.N <= 6144) || (p.M == 4 && p.N <= 2048))) {
        // Three tokens up to three rows per wave, four up to one: the LDS ring
        // reading each row once for every token (3 x 4096 x 1024 / 2048 /
        // 6144: 4.06 / 4.11 / 6.13 us against 4.81 / 4.90 / 6.28 on the
        // skinny tiles, 4096 level at 5.2; 4 x 4096 x 1024 / 2048: 4.51 /
        // 4.69 against 4.89 / 5.04; more rows per wave favour the tiles, 3 x
        // 4096 x 8192 7.24 against 6.62, 4 x 4096 x 4096 5.81 against 5.35).
        const Variant* ring = by_name(p.M == 3 ? "rowlds_m3_r2d1" : "rowlds_m4_r2d1");
        if (ring && gemv_lds_supports(*ring, p)) return ring;
    }
    const bool mid_k = (p.M == 3 || p.M == 4) && p.K > 2048 && p.K < 4096;
    if (p.M == 2 || (p.M == 3 && p.K > 4096 && p.K <= 16384) ||
        (p.M == 4 && p.K > 4096 && p.K <= 16384 && p.K % 1024 != 0) || mid_k) {
        // Rows split over S waves past K = 4096, one workgroup per CU
        // (measured on MI355X: 8192 x 8192 in 9.35 us, 14336 x 4096 in 9.35
        // us, 28672 x 8192 in 26.0 us, against 11.8, 11.8 and 31.4 us for the
        // split-K tiles; three tokens, 8192 x 8192 in 11.1 us and 14336 x
        // 4096 in 11.6 us, against 11.9 and 11.8 us; four tokens where K
        // takes no split-K slicing, 11008 x 4096 in 13.4 us and 13824 x 5120
        // in 15.7 us, against 24.0 and 48.2 us on the vector-ALU GEMV, while
        // where it does the split-K tiles stay ahead, 14336 x 4096 12.1 us
        // against 13.6).  Three or four tokens at 2048 < K < 4096, where
        // the skinny tiles take K in parts of 1024 or no slicing fits: the
        // streaming GEMV reading each row once for all tokens (3 / 4 x 3072 x
        // 8192 in 6.6 / 7.7 us against 10.3 / 10.4 on the split-K tiles; 3 /
        // 4 x 3584 x 18944 in 11.6 / 13.9 against 28.1 / 28.6 on the
        // vector-ALU GEMV).
        uint32_t split = 1;
        while (split < 8 && p.K > 4096u * split) split *= 2;
        if (split == 1 && (p.M == 2 || p.N <= 10240)) {
            // Two tokens at K <= 4096 (K % 256 == 0, 16-byte aligned): the LDS
            // ring reading each row once for both tokens (2 x 4096 x 4096 /
            // 6144 / 14336: 4.25 / 5.11 / 8.37 us, against 4.94 / 6.40 /
            // 9.2 us on the streaming GEMV below).  Three or four tokens at
            // 2048 < K < 4096 up to five rows per wave, bit for bit the
            // streaming GEMV (3 / 4 x 2560 x 10240: 8.17 / 9.48 us against
            // 9.03 / 10.64; 3072 x 8192: 7.14 / 8.30 against 7.38 / 8.53;
            // at 3584 x 18944 the ring is 2-3 % slower).
            const Variant* ring = by_name(p.M == 2 ? "rowlds_m2_r2d1" : p.M == 3 ? "rowlds_m3_r2d1" : "rowlds_m4_r2d1");
            if (ring && gemv_lds_supports(*ring, p)) return ring;
        }
        char name[32];
        if (split == 1 && p.M > 2)
            std::snprintf(name, sizeof name, "%s", p.M == 3 ? "stream_m3_d1_g1" : "stream_m4_d1_g1");
        else if (split == 1)
            std::snprintf(name, sizeof name, "%s", "stream_m2_d1q_g1");
        else
            std::snprintf(name, sizeof name, "stream_s%u_m%u_d1q_g1", split, p.M);
        const Variant* v = by_name(name);
        if (v && gemv_stream_supports(*v, p)) return v;
    }
    if (p.M >= 5 && p.M <= 11 && p.K > 4096 && p.K <= 16384 && p.K % 1024 != 0) {
        // 5-11 tokens where K takes no split-K slicing: passes of up to four
        // tokens on the split-row streaming GEMV (each pass reads the
        // weights once; measured on MI355X: a four-token pass at 11008 x
        // 4096 13.4 us, against 32.7 us for 8 tokens on the vector-ALU GEMV
        // and 40.4 us on the prefill tiles)
        char name[32];
        std::snprintf(name, sizeof name, "stream_s%u_m4x_d1q_g1", p.K > 8192 ? 4u : 2u);
        const Variant* v = by_name(name);
        if (v && gemv_stream_supports(*v, p)) return v;
    }
    if (p.M >= 5 && p.M <= 11 && p.K > 2048 && p.K < 4096 && p.K % 1024 != 0 && p.N >= 8192) {
        // the same with whole rows below K = 4096 (6 / 8 / 11 x 3584 x 18944
        // in 23.4 / 28.2 / 39.6 us against 38.9 / 49.9 / 66.9 on the
        // vector-ALU GEMV; with fewer rows, 6 x 3584 x 4608, that one stays
        // ahead: 12.1 against 13.2)
        const Variant* v = by_name("stream_m4x_d1q_g1");
        if (v && gemv_stream_supports(*v, p)) return v;
    }
    if (const Variant* v = skinny_heuristic(p)) return v;
    if (const Variant* v = split_k(p, op, split_ok)) return v;
    // one K slice of 2048 or 1024 (K that no split fits)
    for (const char* name : {"skinny_mfma_k8_s1_t1_d1_g1_r1", "skinny_mfma_k4_s1_t1_d1_g1_r1"}) {
        const Variant* v = by_name(name);
        if (v && skinny_mfma_supports(*v, p)) return v;
    }
    // 12 tokens and more with no K slicing (K % 1024 != 0, e.g. 11 008 and
    // 13 824): the prefill tiles (measured on MI355X: 16 x 11008 x 4096 in
    // 40.4 us, 32 x 13824 x 5120 in 50.5 us, against 59.0 and 181.3 us on
    // the vector-ALU GEMV; 8 tokens 40.4 / 50.0 against 32.7 / 50.8)
    if (p.M >= 12)
        if (const Variant* v = cheapest_tiles(p, kTiles)) return v;
    // the vector-ALU GEMV one token per pass from 3 tokens (measured on
    // MI355X: 3 / 5 / 11 x 18944 x 3584 in 24.8 / 36.3 / 66.9 us against 28.3
    // / 39.8 / 72.6 with two tokens per pass and 58.6 at 5 with four; 8 x
    // 3584 x 4608: 14.6 against 16.0)
    return by_name(p.M == 2 ? "gemv_r4_t2_k1" : "gemv_r4_t1_k1");
}

// Measured plans for the workloads the path is tuned on (the decode, skinny
// and prefill linears and the fused gate/up at their benchmark shapes): every
// candidate the autotuner would time for the shape, with its kernel time in
// microseconds on MI355X (graph replays, weights rotated past the MALL), as
// written by `bench.py --plan-table`.  A listed shape with operands on the
// 16-byte grid (the class the table was measured in) runs its fastest entry
// that supports the operands; every other shape runs the rules above.
struct PlanEntry {
    int op;  // Op
    uint32_t m, k, n;
    const char* variant;
    double us;
};
constexpr PlanEntry kPlanTable[] = {
#include "plan_table.inc"
    {-1, 0, 0, 0, "", 0.0},  // end
};

const Variant* table_pick(const Problem& p, Op op, bool split_ok) {
    if (align_class(p) != 2) return nullptr;
    const Variant* best = nullptr;
    double best_us = 0.0;
    for (const PlanEntry& e : kPlanTable) {
        if (e.op != static_cast<int>(op) || e.m != p.M || e.k != p.K || e.n != p.N) continue;
        const Variant* v = find_variant(e.variant);
        if (!v || !kind_matches(*v, op) || !supports(*v, p) || (!split_ok && splits_k(*v))) continue;
        if (!best || e.us < best_us) {
            best = v;
            best_us = e.us;
        }
    }
    return best;
}

// The shape heuristic used when autotuning is off: the plan table, then the
// rules.
const Variant* heuristic(const Problem& p, Op op, bool split_ok = true) {
    if (const Variant* v = table_pick(p, op, split_ok)) return v;
    return rules(p, op, split_ok);
}

hipError_t time_variant(const Variant& v, const Problem& p, float* ms) {
    hipEvent_t start = nullptr, stop = nullptr;
    hipError_t err = hipEventCreate(&start);
    if (err == hipSuccess) err = hipEventCreate(&stop);
    if (err == hipSuccess) err = v.launch(p);  // warm-up
    if (err == hipSuccess) err = hipEventRecord(start, p.stream);
    for (int i = 0; i < 5 && err == hipSuccess; ++i) err = v.launch(p);
    if (err == hipSuccess) err = hipEventRecord(stop, p.stream);
    if (err == hipSuccess) err = hipEventSynchronize(stop);
    if (err == hipSuccess) err = hipEventElapsedTime(ms, start, stop);
    if (start) (void)hipEventDestroy(start);
    if (stop) (void)hipEventDestroy(stop);
    return err;
}

int fail(Dispatcher* d, hipError_t status, const std::string& message) {
    if (d) d->last_error = message;
    return static_cast<int>(status);
}

int run(Dispatcher& d, const Problem& problem, Op op) {
    std::lock_guard<std::mutex> lock(d.mutex);
    Problem p = problem;
    p.splitk_fold = d.splitk_fold;
    const Variant* v = nullptr;
    if (!d.forced.empty()) {
        v = find_variant(d.forced);
        if (!v || !kind_matches(*v, op) || !supports(*v, p))
            return fail(&d, hipErrorInvalidValue,
                        "forced Q4_0 variant '" + d.forced + "' cannot run this problem");
    } else {
        const Key key{p.M, p.N, p.K, static_cast<int>(op), static_cast<int>(p.out), align_class(p)};
        auto found = d.plans.find(key);
        if (found == d.plans.end()) {
            const Variant* chosen = nullptr;
            if (d.autotune) {
                float best = 0.0f;
                // the shape heuristic's pick is always among those timed (it
                // may be of a kind the list leaves out for this M, e.g. the
                // prefill tiles for 12-63 tokens where K has no slicing)
                std::vector<const Variant*> cands = candidates(p, op);
                const Variant* h = heuristic(p, op);
                if (h && std::find(cands.begin(), cands.end(), h) == cands.end()) cands.push_back(h);
                for (const Variant* c : cands) {
                    float ms = 0.0f;
                    const hipError_t err = time_variant(*c, p, &ms);
                    if (err != hipSuccess)
                        return fail(&d, err, std::string("autotuning ") + c->name + " failed");
                    if (!chosen || ms < best) {
                        chosen = c;
                        best = ms;
                    }
                }
            }
            if (!chosen) chosen = heuristic(p, op);
            if (!chosen) return fail(&d, hipErrorInvalidValue, "no Q4_0 variant for this problem");
            found = d.plans.emplace(key, chosen).first;
        }
        v = found->second;
        // the key's alignment class already implies this; checked again so
        // that no launch ever runs outside its kernel's stated conditions
        if (!supports(*v, p)) return fail(&d, hipErrorInvalidValue, std::string("cached plan ") + v->name +
                                                                      " cannot run this problem");
    }
    hipError_t err = v->launch(p);
    if (err == hipErrorStreamCaptureUnsupported && splits_k(*v) && d.forced.empty()) {
        // Under graph capture the stream's split-K scratch was too small (a
        // capture may not allocate) and nothing was queued: this call runs
        // the best plan without split K instead (the cached plan stays for
        // eager calls, which size the scratch).
        const Variant* f = heuristic(p, op, false);
        if (f && supports(*f, p)) {
            v = f;
            err = f->launch(p);
        }
    }
    if (err != hipSuccess) return fail(&d, err, std::string("launch of ") + v->name + " failed");
    d.last_error.clear();
    return 0;
}

// The launch of the entry point that allocates nothing: the cached plan, or
// on the first call of a shape the shape heuristic (never the autotuner,
// which would create events and synchronise), then the launch.
int run_no_alloc(Dispatcher& d, const Problem& problem) {
    std::lock_guard<std::mutex> lock(d.mutex);
    Problem p = problem;
    p.splitk_fold = d.splitk_fold;
    const Variant* v = nullptr;
    if (!d.forced.empty()) {
        v = find_variant(d.forced);
        if (!v || !kind_matches(*v, Op::Linear) || !supports(*v, p)) return hipErrorInvalidValue;
    } else {
        const Key key{p.M, p.N, p.K, static_cast<int>(Op::Linear), static_cast<int>(p.out), align_class(p)};
        auto found = d.plans.find(key);
        if (found == d.plans.end()) {
            const Variant* chosen = heuristic(p, Op::Linear);
            if (!chosen) return hipErrorInvalidValue;
            found = d.plans.emplace(key, chosen).first;
        }
        v = found->second;
        if (!supports(*v, p)) return hipErrorInvalidValue;  // as in run(): never outside the kernel's conditions
    }
    return static_cast<int>(v->launch(p));
}

Dispatcher& default_dispatcher() {
    static Dispatcher* d = [] {
        auto* x = new Dispatcher();
        const char* tune = std::getenv("MOTE_Q4_0_AUTOTUNE");
        x->autotune = tune && tune[0] == '1';
        const char* forced = std::getenv("MOTE_Q4_0_VARIANT");
        if (forced) x->forced = forced;
        return x;
    }();
    return *d;
}

// Argument checks shared by every linear entry point, in the reference order
// (crates/mote-backend-hip/src/quantized_linear.hip:64-76).  Returns -1 when
// the caller should go on and launch, otherwise the status to return.
int check_linear(const void* input, const void* weights, const void* output, uint64_t rows,
                 uint64_t n, uint64_t k, const void* stream) {
    if (!input || !weights || !output || !stream) return hipErrorInvalidValue;
    if (k % 32 != 0) return hipErrorInvalidValue;
    if (rows == 0 || n == 0) return hipSuccess;
    if (rows > UINT_MAX || n > UINT_MAX || rows > UINT_MAX / n) return hipErrorInvalidConfiguration;
    return -1;
}

// The largest K of the tiled kernels (32-bit K and element offsets); larger K
// runs the 64-bit path of q4_0_wide_k.hip, outside the plans.
constexpr uint64_t kMaxTiledK = 0x7fffffffull;

int wide(Dispatcher* d, const Problem& problem, uint64_t k, bool q8) {
    Dispatcher& disp = d ? *d : default_dispatcher();
    std::lock_guard<std::mutex> lock(disp.mutex);
    if (!disp.forced.empty())
        return fail(d, hipErrorInvalidValue, "forced Q4_0 variant '" + disp.forced + "' cannot run K > 2^31 - 1");
    const hipError_t e = launch_wide_k(problem, k, q8);
    return e == hipSuccess ? 0 : fail(d, e, "wide-K launch failed");
}

int linear(Dispatcher* d, const void* input, const void* weights, void* output, uint64_t rows,
           uint64_t n, uint64_t k, OutType out, void* stream, Op op = Op::Linear) {
    const int pre = check_linear(input, weights, output, rows, n, k, stream);
    if (pre >= 0) return pre == 0 ? 0 : fail(d, static_cast<hipError_t>(pre), "invalid quantized linear arguments");
    const auto s = static_cast<hipStream_t>(stream);
    if (k == 0) return static_cast<int>(launch_zero_fill(output, rows * n, out, s));
    if (k > kMaxTiledK)
        return wide(d, Problem{input, weights, nullptr, output, static_cast<uint32_t>(rows), static_cast<uint32_t>(n),
                               0, out, s},
                    k, op == Op::LinearQ8);
    const Problem p{input, weights, nullptr, output, static_cast<uint32_t>(rows),
                    static_cast<uint32_t>(n), static_cast<uint32_t>(k), out, s};
    return run(d ? *d : default_dispatcher(), p, op);
}

int gate_up(Dispatcher* d, const void* input, const void* gate, const void* up, void* output,
            uint64_t rows, uint64_t n, uint64_t k, OutType out, void* stream) {
    const int pre = check_linear(input, gate, output, rows, n, k, stream);
    if (pre >= 0) return pre == 0 ? 0 : fail(d, static_cast<hipError_t>(pre), "invalid Q4_0 gate/up arguments");
    const auto s = static_cast<hipStream_t>(stream);
    if (k == 0) return static_cast<int>(launch_zero_fill(output, rows * n, out, s));
    if (up == nullptr) up = static_cast<const uint8_t*>(gate) + n * (k / 32) * 18;
    if (k > kMaxTiledK)
        return wide(d, Problem{input, gate, up, output, static_cast<uint32_t>(rows), static_cast<uint32_t>(n), 0, out, s},
                    k, false);
    const Problem p{input, gate, up, output, static_cast<uint32_t>(rows), static_cast<uint32_t>(n),
                    static_cast<uint32_t>(k), out, s};
    return run(d ? *d : default_dispatcher(), p, Op::GateUp);
}

}  // namespace

namespace {

// Scratch of destroyed streams, parked until the work queued before the
// destroy has completed: the buffers and an event recorded on the stream
// just before it was destroyed.
struct Parked {
    hipEvent_t done;
    std::vector<void*> buffers;
};
std::mutex g_parked_mu;
std::vector<Parked>* g_parked = new std::vector<Parked>;  // lives until exit

// Frees the parked buffers whose event has completed (a free that fails is
// reported through the return value; its buffers are dropped either way).
hipError_t reap_parked() {
    std::lock_guard<std::mutex> lock(g_parked_mu);
    hipError_t status = hipSuccess;
    for (auto it = g_parked->begin(); it != g_parked->end();) {
        const hipError_t q = hipEventQuery(it->done);
        if (q == hipErrorNotReady) {
            ++it;
            continue;
        }
        for (void* p : it->buffers) {
            const hipError_t f = hipFree(p);
            if (status == hipSuccess) status = f;
        }
        (void)hipEventDestroy(it->done);
        if (status == hipSuccess && q != hipSuccess) status = q;
        it = g_parked->erase(it);
    }
    return status;
}

// Called only when the pool needs a new buffer, which never happens under
// graph capture (an allocation there would fail anyway), so the event
// queries of reap_parked() never run inside a capture.
int device_alloc(void** ptr, size_t bytes) {
    (void)reap_parked();
    return static_cast<int>(hipMalloc(ptr, bytes));
}
int device_free(void* ptr) { return static_cast<int>(hipFree(ptr)); }

ScratchPool& scratch_pool() {
    static ScratchPool* pool = new ScratchPool(device_alloc, device_free);  // lives until exit
    return *pool;
}

}  // namespace

hipError_t acquire_scratch(hipStream_t stream, size_t bytes, ScratchPool::Lease* lease) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    // A stream under graph capture must not allocate: its buffer is used if
    // it is large enough, else hipErrorStreamCaptureUnsupported before any
    // launch.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &capture);
    if (e != hipSuccess) return e;
    const int status = scratch_pool().acquire(dev, stream, bytes, lease, capture == hipStreamCaptureStatusNone);
    if (status == ScratchPool::kWouldAllocate) return hipErrorStreamCaptureUnsupported;
    return static_cast<hipError_t>(status);
}

hipError_t reserve_stream_scratch(hipStream_t stream, size_t bytes) {
    ScratchPool::Lease lease;
    const hipError_t e = acquire_scratch(stream, bytes, &lease);
    if (e != hipSuccess) return e;
    if (!lease.fresh()) return hipSuccess;
    // a new buffer: its split-K tile counters start at zero
    return launch_zero_fill(lease.ptr(), kSplitKCounterBytes / 4, OutType::F32, stream);
}

hipError_t reap_parked_scratch() { return reap_parked(); }

hipError_t park_stream_scratch(hipStream_t stream) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::vector<void*> buffers = scratch_pool().detach(dev, stream);
    if (buffers.empty()) return reap_parked();
    hipEvent_t done = nullptr;
    e = hipEventCreateWithFlags(&done, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(done, stream);
    if (e != hipSuccess) {
        // no completion point to wait for: wait for the stream instead
        if (done != nullptr) (void)hipEventDestroy(done);
        const hipError_t sync = hipStreamSynchronize(stream);
        const hipError_t freed = static_cast<hipError_t>(scratch_pool().free_all(buffers));
        return sync != hipSuccess ? sync : (freed != hipSuccess ? freed : e);
    }
    {
        std::lock_guard<std::mutex> lock(g_parked_mu);
        g_parked->push_back(Parked{done, std::move(buffers)});
    }
    return reap_parked();
}

}  // namespace mote::q4_0

using namespace mote::q4_0;

namespace {

// Split-K scratch of mote_hip_quantized_linear_q4_0_f32_no_alloc: a
// file-scope device array, so the entry point never allocates.  Every GPU
// that loads the library holds its own copy until the process ends.  In host
// code the name `scratch` is only a stand-in for the symbol, not a device
// address: the address each device's copy has is fetched once per device
// with hipGetSymbolAddress and only that address is passed to kernels.
constexpr size_t kNoAllocScratchBytes = size_t{16} << 20;
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

// The current device's address of `scratch`, fetched on the first call on
// that device (with the device current) and kept.
hipError_t no_alloc_scratch(void** ptr) {
    static std::mutex mu;
    static void* addresses[64] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (addresses[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        addresses[dev] = p;
    }
    *ptr = addresses[dev];
    return hipSuccess;
}

}  // namespace

MOTE_EXPORT int mote_hip_quantized_linear_q4_0_f16(const void* input, const void* weights,
                                                  void* output, uint64_t rows,
                                                  uint64_t output_features,
                                                  uint64_t input_features, void* stream) noexcept {
    try {
        return linear(nullptr, input, weights, output, rows, output_features, input_features,
                      OutType::F16, stream);
    } catch (...) {
        return hipErrorUnknown;
    }
}

MOTE_EXPORT int mote_hip_quantized_linear_q4_0_f32(const void* input, const void* weights,
                                                  void* output, uint64_t rows,
                                                  uint64_t output_features,
                                                  uint64_t input_features, void* stream) noexcept {
    try {
        return linear(nullptr, input, weights, output, rows, output_features, input_features,
                      OutType::F32, stream);
    } catch (...) {
        return hipErrorUnknown;
    }
}

// mote_hip_quantized_linear_q4_0_f32 for callers that cannot allocate (code
// under graph capture, serving loops that forbid hipMalloc): the same
// checks, plans and kernels, with the split-K partial tiles in the library's
// static 16 MiB device array instead of the per-stream pool.  Calls on one
// GPU share that array, so calls that overlap in time on one GPU (other
// streams, other threads) race; a problem whose partial tiles exceed it
// returns hipErrorOutOfMemory (2) before any launch.
MOTE_EXPORT int mote_hip_quantized_linear_q4_0_f32_no_alloc(const void* input, const void* weights,
                                                           void* output, uint64_t rows,
                                                           uint64_t output_features,
                                                           uint64_t input_features, void* stream) noexcept {
    try {
        const int pre = check_linear(input, weights, output, rows, output_features, input_features, stream);
        if (pre >= 0) return pre;
        const auto s = static_cast<hipStream_t>(stream);
        if (input_features == 0) return static_cast<int>(launch_zero_fill(output, rows * output_features, OutType::F32, s));
        void* buf = nullptr;
        const hipError_t e = no_alloc_scratch(&buf);
        if (e != hipSuccess) return static_cast<int>(e);
        Problem p{input, weights, nullptr, output, static_cast<uint32_t>(rows), static_cast<uint32_t>(output_features),
                  input_features > kMaxTiledK ? 0u : static_cast<uint32_t>(input_features), OutType::F32, s};
        p.scratch = static_cast<float*>(buf);
        p.scratch_bytes = kNoAllocScratchBytes;
        if (input_features > kMaxTiledK) {
            Dispatcher& d = default_dispatcher();
            std::lock_guard<std::mutex> lock(d.mutex);
            if (!d.forced.empty()) return hipErrorInvalidValue;
            return static_cast<int>(launch_wide_k(p, input_features, false));
        }
        return run_no_alloc(default_dispatcher(), p);
    } catch (...) {
        return hipErrorUnknown;
    }
}

MOTE_EXPORT int mote_hip_quantized_linear_q8_0_f16(const void* input, const void* weights,
                                                  void* output, uint64_t rows,
                                                  uint64_t output_features,
                                                  uint64_t input_features, void* stream) noexcept {
    try {
        return linear(nullptr, input, weights, output, rows, output_features, input_features,
                      OutType::F16, stream, Op::LinearQ8);
    } catch (...) {
        return hipErrorUnknown;
    }
}

MOTE_EXPORT int mote_hip_quantized_linear_q8_0_f32(const void* input, const void* weights,
                                                  void* output, uint64_t rows,
                                                  uint64_t output_features,
                                                  uint64_t input_features, void* stream) noexcept {
    try {
        return linear(nullptr, input, weights, output, rows, output_features, input_features,
                      OutType::F32, stream, Op::LinearQ8);
    } catch (...) {
        return hipErrorUnknown;
    }
}

MOTE_EXPORT int mote_hip_q4_0_gate_up_silu_f32(const void* input, const void* gate_weights,
                                              const void* up_weights, void* output,
                                              uint64_t rows, uint64_t output_features,
                                              uint64_t input_features, void* stream) noexcept {
    try {
        return gate_up(nullptr, input, gate_weights, up_weights, output, rows, output_features,
                       input_features, OutType::F32, stream);
    } catch (...) {
        return hipErrorUnknown;
    }
}

MOTE_EXPORT int mote_hip_dequantize_q4_0_f32(const void* weights, void* output, uint64_t rows,
                                            uint64_t input_features, void* stream) noexcept {
    if (!weights || !output || !stream) return hipErrorInvalidValue;
    if (input_features % 32 != 0) return hipErrorInvalidValue;
    if (rows == 0 || input_features == 0) return hipSuccess;
    if (rows > (1ull << 40) / input_features) return hipErrorInvalidConfiguration;
    return static_cast<int>(launch_decode_f32(weights, static_cast<float*>(output), rows,
                                              input_features, static_cast<hipStream_t>(stream)));
}

MOTE_EXPORT int mote_q4_0_dispatch_create(void** handle) noexcept {
    if (!handle) return hipErrorInvalidValue;
    *handle = nullptr;
    try {
        *handle = new mote::q4_0::Dispatcher();
        return 0;
    } catch (...) {
        return hipErrorOutOfMemory;
    }
}

MOTE_EXPORT void mote_q4_0_dispatch_destroy(void* handle) noexcept {
    delete static_cast<mote::q4_0::Dispatcher*>(handle);
}

MOTE_EXPORT const char* mote_q4_0_dispatch_last_error(void* handle) noexcept {
    auto* d = static_cast<mote::q4_0::Dispatcher*>(handle);
    return d ? d->last_error.c_str() : nullptr;
}

MOTE_EXPORT int mote_q4_0_dispatch_set_autotune(void* handle, int enabled) noexcept {
    auto* d = static_cast<mote::q4_0::Dispatcher*>(handle);
    if (!d) return hipErrorInvalidValue;
    std::lock_guard<std::mutex> lock(d->mutex);
    d->autotune = enabled != 0;
    return 0;
}

MOTE_EXPORT int mote_q4_0_dispatch_set_splitk_fold(void* handle, int enabled) noexcept {
    auto* d = static_cast<mote::q4_0::Dispatcher*>(handle);
    if (!d) return hipErrorInvalidValue;
    std::lock_guard<std::mutex> lock(d->mutex);
    d->splitk_fold = enabled != 0;
    return 0;
}

MOTE_EXPORT int mote_q4_0_dispatch_force_variant(void* handle, const char* name) noexcept {
    auto* d = static_cast<mote::q4_0::Dispatcher*>(handle);
    if (!d) return hipErrorInvalidValue;
    std::lock_guard<std::mutex> lock(d->mutex);
    if (name == nullptr || name[0] == '\0') {
        d->forced.clear();
        return 0;
    }
    if (!find_variant(name)) {
        d->last_error = std::string("unknown Q4_0 variant '") + name + "'";
        return hipErrorInvalidValue;
    }
    d->forced = name;
    return 0;
}

MOTE_EXPORT int mote_q4_0_dispatch_linear(void* handle, const void* input, const void* weights,
                                         void* output, uint64_t rows, uint64_t output_features,
                                         uint64_t input_features, int output_f16,
                                         void* stream) noexcept {
    auto* d = static_cast<mote::q4_0::Dispatcher*>(handle);
    if (!d) return hipErrorInvalidValue;
    try {
        return linear(d, input, weights, output, rows, output_features, input_features,
                      output_f16 ? OutType::F16 : OutType::F32, stream);
    } catch (...) {
        return fail(d, hipErrorUnknown, "unexpected C++ exception");
    }
}

MOTE_EXPORT int mote_q4_0_dispatch_linear_q8_0(void* handle, const void* input, const void* weights,
                                              void* output, uint64_t rows, uint64_t output_features,
                                              uint64_t input_features, int output_f16,
                                              void* stream) noexcept {
    auto* d = static_cast<mote::q4_0::Dispatcher*>(handle);
    if (!d) return hipErrorInvalidValue;
    try {
        return linear(d, input, weights, output, rows, output_features, input_features,
                      output_f16 ? OutType::F16 : OutType::F32, stream, Op::LinearQ8);
    } catch (...) {
        return fail(d, hipErrorUnknown, "unexpected C++ exception");
    }
}

MOTE_EXPORT int mote_q4_0_dispatch_gate_up_silu(void* handle, const void* input,
                                               const void* gate_weights, const void* up_weights,
                                               void* output, uint64_t rows,
                                               uint64_t output_features, uint64_t input_features,
                                               int output_f16, void* stream) noexcept {
    auto* d = static_cast<mote::q4_0::Dispatcher*>(handle);
    if (!d) return hipErrorInvalidValue;
    try {
        return gate_up(d, input, gate_weights, up_weights, output, rows, output_features,
                       input_features, output_f16 ? OutType::F16 : OutType::F32, stream);
    } catch (...) {
        return fail(d, hipErrorUnknown, "unexpected C++ exception");
    }
}

MOTE_EXPORT int mote_q4_0_dispatch_plan(void* handle, uint64_t rows, uint64_t output_features,
                                       uint64_t input_features, int gate_up_op, int output_f16,
                                       char* name, size_t capacity) noexcept {
    auto* d = static_cast<mote::q4_0::Dispatcher*>(handle);
    if (!d || !name || capacity == 0) return hipErrorInvalidValue;
    std::lock_guard<std::mutex> lock(d->mutex);
    for (const auto& entry : d->plans) {
        const auto& k = entry.first;
        if (k.m == rows && k.n == output_features && k.k == input_features &&
            k.op == gate_up_op && k.out == output_f16) {
            std::strncpy(name, entry.second->name, capacity - 1);
            name[capacity - 1] = '\0';
            return 0;
        }
    }
    name[0] = '\0';
    return hipErrorNotFound;
}

MOTE_EXPORT int mote_q4_0_dispatch_select(void* handle, uint64_t rows, uint64_t output_features,
                                         uint64_t input_features, int op, char* name, size_t capacity) noexcept {
    auto* d = static_cast<mote::q4_0::Dispatcher*>(handle);
    if (!d || !name || capacity == 0 || op < 0 || op > 2) return hipErrorInvalidValue;
    name[0] = '\0';
    if (rows == 0 || output_features == 0 || input_features == 0 || input_features % 32 != 0 ||
        rows > UINT_MAX || output_features > UINT_MAX)
        return hipErrorInvalidValue;
    try {
        if (input_features > kMaxTiledK) {  // the 64-bit path, which no variant name forces
            std::lock_guard<std::mutex> lock(d->mutex);
            if (!d->forced.empty()) return hipErrorNotFound;
            std::strncpy(name, "wide_k", capacity - 1);
            name[capacity - 1] = '\0';
            return 0;
        }
        // Stand-in operands at the library's 256-byte allocation alignment;
        // nothing is dereferenced or launched.
        const auto* base = reinterpret_cast<const uint8_t*>(uintptr_t{1} << 20);
        const Problem p{base, base, op == static_cast<int>(Op::GateUp) ? base : nullptr, const_cast<uint8_t*>(base),
                        static_cast<uint32_t>(rows), static_cast<uint32_t>(output_features),
                        static_cast<uint32_t>(input_features), OutType::F32, nullptr};
        std::lock_guard<std::mutex> lock(d->mutex);
        const Variant* v = d->forced.empty() ? heuristic(p, static_cast<Op>(op)) : find_variant(d->forced);
        if (!v) return hipErrorNotFound;
        std::strncpy(name, v->name, capacity - 1);
        name[capacity - 1] = '\0';
        return 0;
    } catch (...) {
        return hipErrorUnknown;
    }
}

MOTE_EXPORT int mote_q4_0_dispatch_candidates(void* handle, uint64_t rows, uint64_t output_features,
                                             uint64_t input_features, int op, char* names, size_t capacity) noexcept {
    auto* d = static_cast<mote::q4_0::Dispatcher*>(handle);
    if (!d || !names || capacity == 0 || op < 0 || op > 2) return hipErrorInvalidValue;
    names[0] = '\0';
    if (rows == 0 || output_features == 0 || input_features == 0 || input_features % 32 != 0 ||
        rows > UINT_MAX || output_features > UINT_MAX || input_features > 0x7fffffffull)
        return hipErrorInvalidValue;
    try {
        const auto* base = reinterpret_cast<const uint8_t*>(uintptr_t{1} << 20);
        const Problem p{base, base, op == static_cast<int>(Op::GateUp) ? base : nullptr, const_cast<uint8_t*>(base),
                        static_cast<uint32_t>(rows), static_cast<uint32_t>(output_features),
                        static_cast<uint32_t>(input_features), OutType::F32, nullptr};
        std::lock_guard<std::mutex> lock(d->mutex);
        std::vector<const Variant*> cands = candidates(p, static_cast<Op>(op));
        const Variant* r = rules(p, static_cast<Op>(op), true);
        if (r && std::find(cands.begin(), cands.end(), r) == cands.end()) cands.push_back(r);
        std::string out;
        for (const Variant* v : cands) {
            if (!out.empty()) out += ',';
            out += v->name;
        }
        if (out.size() + 1 > capacity) return hipErrorInvalidValue;
        std::memcpy(names, out.c_str(), out.size() + 1);
        return 0;
    } catch (...) {
        return hipErrorUnknown;
    }
}

MOTE_EXPORT int mote_q4_0_variant_count(void) noexcept {
    return static_cast<int>(all_variants().size());
}

MOTE_EXPORT const char* mote_q4_0_variant_name(int index) noexcept {
    const auto v = all_variants();
    return (index >= 0 && index < static_cast<int>(v.size())) ? v[static_cast<size_t>(index)]->name
                                                             : nullptr;
}

// Host-side interface between the Q4_0 launch entry points, the dispatch cache
// and the kernels.  Nothing here is part of the exported C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "scratch_pool.hpp"

namespace mote::q4_0 {

enum class OutType : int { F32 = 0, F16 = 1 };

struct Problem {
    const void* x;        // f16 [M, K]
    const void* w;        // Q4_0 [N, K] (Q8_0 for the Q8_0 linear; gate rows for the fused op)
    const void* w_up;     // Q4_0 [N, K]  up rows, fused gate/up only (else null)
    void* y;              // [M, N] f32 or f16
    uint32_t M, N, K;
    OutType out;
    hipStream_t stream;
    // Caller-provided split-K scratch (device memory of scratch_bytes); null:
    // the stream's buffer from the library's scratch pool.
    float* scratch = nullptr;
    size_t scratch_bytes = 0;
    // Split K: the tiles kernel adds the K parts itself (the last workgroup
    // of a tile to finish) instead of a second kernel.  Off by default: on
    // MI355X the fold measured slower (its workgroups wait for their
    // write-through partial stores and the arrival atomic before exiting).
    bool splitk_fold = false;
};

// Split-K scratch layout: kSplitKCounterBytes of per-tile arrival counters
// (zero between calls: the workgroup that adds a tile's parts resets its
// counter) followed by the partial tiles.
constexpr size_t kSplitKCounterBytes = 64 * 1024;

enum class Kind : int { Gemv = 0, Mfma = 1, Generic = 2, GateUpMfma = 3, GateUpGeneric = 4, GemvRows = 5,
                        GemvStream = 6, SkinnyMfma = 7, Q8Stream = 8, Q8Generic = 9, GateUpSkinny = 10,
                        GateUpStream = 11, Q8Skinny = 12, Q8Prefill = 13, GemvLds = 14,
                        Q8Lds = 15 };

struct Variant {
    const char* name;
    Kind kind;
    int p0, p1, p2;       // kernel tile parameters (meaning depends on kind)
    hipError_t (*launch)(const Problem&);
    int tokens = 0;       // exact M the variant requires (0: any M it supports)
};

// Kernel variant tables, defined next to the kernels.
const Variant* gemv_variants(int* count);
const Variant* gemv_rows_variants(int* count);
const Variant* gemv_stream_variants(int* count);
const Variant* gemv_lds_variants(int* count);
const Variant* skinny_mfma_variants(int* count);
const Variant* prefill_variants(int* count);
const Variant* generic_variants(int* count);

// Whether a variant can run the problem (alignment, shape limits).
bool gemv_supports(const Variant& v, const Problem& p);
bool gemv_rows_supports(const Variant& v, const Problem& p);
bool gemv_stream_supports(const Variant& v, const Problem& p);
bool gemv_lds_supports(const Variant& v, const Problem& p);
bool skinny_mfma_supports(const Variant& v, const Problem& p);
bool prefill_supports(const Variant& v, const Problem& p);

hipError_t launch_zero_fill(void* y, uint64_t count, OutType out, hipStream_t stream);
// K above 2^31 - 1 (p.K unused; the fused gate/up when p.w_up is set): 64-bit
// per-element products over K parts of each output, then the parts added in
// part order.  The partials use the split-K scratch (p.scratch when set).
hipError_t launch_wide_k(const Problem& p, uint64_t k, bool q8);

// Split-K scratch owned by the library, one buffer per (device, stream)
// (scratch_pool.hpp): the lease holds the stream's scratch lock, so a caller
// queues every kernel that uses the buffer before the lease goes out of
// scope.  Growing a buffer allocates, which a stream under graph capture may
// not do: there an acquire beyond the buffer's size returns
// hipErrorStreamCaptureUnsupported and allocates nothing.
hipError_t acquire_scratch(hipStream_t stream, size_t bytes, ScratchPool::Lease* lease);
// Sizes a stream's scratch to at least `bytes` ahead of its first split-K
// call (a new buffer gets its tile counters cleared on the stream).
hipError_t reserve_stream_scratch(hipStream_t stream, size_t bytes);
// Frees the parked scratch of destroyed streams whose work has completed.
hipError_t reap_parked_scratch();
// Forgets a stream's scratch without waiting for its queued work: the buffers
// are parked with an event recorded on the stream and freed once it has
// completed (checked here, at later stream destroys and before the pool next
// allocates).
hipError_t park_stream_scratch(hipStream_t stream);
hipError_t launch_decode_f32(const void* w, float* out, uint64_t rows, uint64_t cols,
                             hipStream_t stream);

}  // namespace mote::q4_0

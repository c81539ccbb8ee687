// HIP runtime wrappers of the C ABI.  Same symbols, arguments and status
// convention as crates/mote-backend-hip/src/hipblaslt_shim.cpp:259-324 (bound
// by crates/mote-backend-hip/src/ffi.rs:42-61): the raw hipError_t as an int,
// 0 on success, -1 for a null out-parameter.  Streams are opaque void*.
#include <hip/hip_runtime.h>

#include "export.hpp"
#include "q4_0.hpp"

#include <cstddef>

namespace {
constexpr int kInvalidArgument = -1;
}

MOTE_EXPORT int mote_hip_get_device_count(int* count) noexcept {
    if (count == nullptr) return kInvalidArgument;
    return static_cast<int>(hipGetDeviceCount(count));
}

MOTE_EXPORT int mote_hip_set_device(int ordinal) noexcept {
    return static_cast<int>(hipSetDevice(ordinal));
}

MOTE_EXPORT int mote_hip_malloc(void** pointer, std::size_t bytes) noexcept {
    if (pointer == nullptr) return kInvalidArgument;
    *pointer = nullptr;
    return static_cast<int>(hipMalloc(pointer, bytes));
}

MOTE_EXPORT int mote_hip_free(void* pointer) noexcept {
    return static_cast<int>(hipFree(pointer));
}

MOTE_EXPORT int mote_hip_memcpy_host_to_device(void* destination, const void* source,
                                              std::size_t bytes) noexcept {
    return static_cast<int>(hipMemcpy(destination, source, bytes, hipMemcpyHostToDevice));
}

MOTE_EXPORT int mote_hip_memcpy_device_to_host(void* destination, const void* source,
                                              std::size_t bytes) noexcept {
    return static_cast<int>(hipMemcpy(destination, source, bytes, hipMemcpyDeviceToHost));
}

// Split-K scratch each stream created here gets up front: the partial tiles
// of every split-K shape up to 64 tokens of a 70B-class MLP (64 x 28 672 x
// 8192 fused gate/up: 58.7 MB), so split-K calls on the stream allocate
// nothing up to that size, under graph capture too.
constexpr std::size_t kStreamScratchBytes = std::size_t{64} << 20;

// As in the reference (crates/mote-backend-hip/src/hipblaslt_shim.cpp:296-305),
// plus the stream's split-K scratch; a stream whose scratch cannot be
// allocated is destroyed again and the error returned.
MOTE_EXPORT int mote_hip_stream_create(void** stream) noexcept {
    if (stream == nullptr) return kInvalidArgument;
    *stream = nullptr;
    hipStream_t native = nullptr;
    hipError_t status = hipStreamCreate(&native);
    if (status != hipSuccess) return static_cast<int>(status);
    try {
        status = mote::q4_0::reserve_stream_scratch(native, kStreamScratchBytes);
    } catch (...) {
        status = hipErrorUnknown;
    }
    if (status != hipSuccess) {
        try {
            (void)mote::q4_0::park_stream_scratch(native);
        } catch (...) {
        }
        (void)hipStreamDestroy(native);
        return static_cast<int>(status);
    }
    *stream = native;
    return 0;
}

// Destroys the stream without waiting for its queued work, as the reference
// does (crates/mote-backend-hip/src/hipblaslt_shim.cpp:307).  The split-K
// scratch the library keeps for the stream is detached first, so a stream
// created later at the same address starts without it, and freed once the
// work queued before the destroy has completed (an event recorded on the
// stream marks that point).
MOTE_EXPORT int mote_hip_stream_destroy(void* stream) noexcept {
    const auto s = static_cast<hipStream_t>(stream);
    hipError_t status = hipSuccess;
    try {
        status = mote::q4_0::park_stream_scratch(s);
    } catch (...) {
        status = hipErrorUnknown;
    }
    const hipError_t destroyed = hipStreamDestroy(s);
    return static_cast<int>(status != hipSuccess ? status : destroyed);
}

// As in the reference; afterwards the parked scratch of destroyed streams
// whose work has completed is freed.
MOTE_EXPORT int mote_hip_stream_synchronize(void* stream) noexcept {
    const hipError_t status = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    if (status == hipSuccess) {
        try {
            (void)mote::q4_0::reap_parked_scratch();
        } catch (...) {
        }
    }
    return static_cast<int>(status);
}

MOTE_EXPORT int mote_hip_mem_get_info(std::size_t* free_bytes, std::size_t* total_bytes) noexcept {
    if (free_bytes == nullptr || total_bytes == nullptr) return kInvalidArgument;
    *free_bytes = 0;
    *total_bytes = 0;
    return static_cast<int>(hipMemGetInfo(free_bytes, total_bytes));
}

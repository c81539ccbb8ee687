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

MOTE_EXPORT int mote_hip_stream_create(void** stream) noexcept {
    if (stream == nullptr) return kInvalidArgument;
    *stream = nullptr;
    hipStream_t native = nullptr;
    const hipError_t status = hipStreamCreate(&native);
    *stream = native;
    return static_cast<int>(status);
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

MOTE_EXPORT int mote_hip_stream_synchronize(void* stream) noexcept {
    return static_cast<int>(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
}

MOTE_EXPORT int mote_hip_mem_get_info(std::size_t* free_bytes, std::size_t* total_bytes) noexcept {
    if (free_bytes == nullptr || total_bytes == nullptr) return kInvalidArgument;
    *free_bytes = 0;
    *total_bytes = 0;
    return static_cast<int>(hipMemGetInfo(free_bytes, total_bytes));
}

// Dense F16 x F16 -> F32 matmul behind the reference's hipBLASLt boundary.
//
// The reference exports mote_hipblaslt_{create, destroy, last_error,
// matmul_f16_f32} (crates/mote-backend-hip/src/hipblaslt_shim.cpp:326-408,
// bound at crates/mote-backend-hip/src/ffi.rs:329-417) for
// matmul_f16_f32 (crates/mote-backend-hip/src/matmul.rs:10-52): row-major
// C[m, n] = A[m, k] B[k, n] with f16 operands, f32 accumulation and output,
// on the caller's stream, with a caller-owned workspace.  A plain dense GEMM
// is a library GEMM, so this file does no arithmetic of its own: it keeps
// the reference's contract (a context per caller, one plan per (m, n, k),
// the first call for a shape timing the library's heuristic candidates and
// keeping the fastest, later calls only enqueueing it; statuses are hipBLAS
// statuses, -1 for argument and internal errors, -1000 - hipError for HIP
// runtime failures, with a message in last_error).
//
// hipBLASLt is opened on first use (dlopen, RTLD_LOCAL), so the quantized
// kernels of this library never load it.  Row-major C = A B is column-major
// C^T = B^T A^T: the library's first operand is B (n x k, leading dim n), its
// second A (k x m, leading dim k) and its output C (n x m, leading dim n), no
// transposes.
#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <cmath>
#include <cstdint>
#include <limits>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <tuple>

#include "export.hpp"

namespace mote::dense {
namespace {

constexpr int kArgumentError = -1;
constexpr int kCandidates = 32;

// The hipBLASLt entry points this file calls, resolved once per process.
struct Library {
    decltype(&hipblasLtCreate) create = nullptr;
    decltype(&hipblasLtDestroy) destroy = nullptr;
    decltype(&hipblasLtMatmulDescCreate) desc_create = nullptr;
    decltype(&hipblasLtMatmulDescDestroy) desc_destroy = nullptr;
    decltype(&hipblasLtMatrixLayoutCreate) layout_create = nullptr;
    decltype(&hipblasLtMatrixLayoutDestroy) layout_destroy = nullptr;
    decltype(&hipblasLtMatmulPreferenceCreate) pref_create = nullptr;
    decltype(&hipblasLtMatmulPreferenceSetAttribute) pref_set = nullptr;
    decltype(&hipblasLtMatmulPreferenceDestroy) pref_destroy = nullptr;
    decltype(&hipblasLtMatmulAlgoGetHeuristic) heuristic = nullptr;
    decltype(&hipblasLtMatmul) matmul = nullptr;
    std::string error;  // empty when every entry point resolved
};

template <typename F>
bool resolve(void* handle, const char* name, F& out, std::string& error) {
    out = reinterpret_cast<F>(dlsym(handle, name));
    if (out == nullptr && error.empty()) error = std::string("hipBLASLt lacks ") + name;
    return out != nullptr;
}

const Library& library() {
    static const Library lib = [] {
        Library l;
        void* handle = nullptr;
        for (const char* path : {"libhipblaslt.so.1", "libhipblaslt.so", "/opt/rocm/lib/libhipblaslt.so.1"}) {
            handle = dlopen(path, RTLD_NOW | RTLD_LOCAL);
            if (handle != nullptr) break;
        }
        if (handle == nullptr) {
            const char* why = dlerror();
            l.error = std::string("cannot load hipBLASLt: ") + (why ? why : "not found");
            return l;
        }
        resolve(handle, "hipblasLtCreate", l.create, l.error);
        resolve(handle, "hipblasLtDestroy", l.destroy, l.error);
        resolve(handle, "hipblasLtMatmulDescCreate", l.desc_create, l.error);
        resolve(handle, "hipblasLtMatmulDescDestroy", l.desc_destroy, l.error);
        resolve(handle, "hipblasLtMatrixLayoutCreate", l.layout_create, l.error);
        resolve(handle, "hipblasLtMatrixLayoutDestroy", l.layout_destroy, l.error);
        resolve(handle, "hipblasLtMatmulPreferenceCreate", l.pref_create, l.error);
        resolve(handle, "hipblasLtMatmulPreferenceSetAttribute", l.pref_set, l.error);
        resolve(handle, "hipblasLtMatmulPreferenceDestroy", l.pref_destroy, l.error);
        resolve(handle, "hipblasLtMatmulAlgoGetHeuristic", l.heuristic, l.error);
        resolve(handle, "hipblasLtMatmul", l.matmul, l.error);
        return l;  // the handle stays open for the life of the process
    }();
    return lib;
}

// One shape's descriptors and chosen algorithm.
struct Plan {
    hipblasLtMatmulDesc_t op = nullptr;
    hipblasLtMatrixLayout_t b_layout = nullptr, a_layout = nullptr, c_layout = nullptr;
    hipblasLtMatmulAlgo_t algo{};

    ~Plan() {
        const Library& l = library();
        if (c_layout) l.layout_destroy(c_layout);
        if (a_layout) l.layout_destroy(a_layout);
        if (b_layout) l.layout_destroy(b_layout);
        if (op) l.desc_destroy(op);
    }
};

struct Context {
    hipblasLtHandle_t handle = nullptr;
    std::mutex mutex;
    std::map<std::tuple<uint64_t, uint64_t, uint64_t>, std::unique_ptr<Plan>> plans;
    std::string last_error;

    ~Context() {
        plans.clear();
        if (handle) library().destroy(handle);
    }

    int fail(int status, const std::string& what) {
        last_error = what;
        return status == 0 ? kArgumentError : status;
    }
    int fail_blas(hipblasStatus_t status, const char* what) {
        return fail(static_cast<int>(status), std::string(what) + " failed (hipBLAS status " +
                                                  std::to_string(static_cast<int>(status)) + ")");
    }
    int fail_hip(hipError_t status, const char* what) {
        return fail(-1000 - static_cast<int>(status), std::string(what) + " failed: " + hipGetErrorString(status));
    }
};

// Enqueues C^T = B^T A^T with `plan`'s algorithm.
hipblasStatus_t enqueue(const Context& ctx, const Plan& plan, const void* a, const void* b, void* c,
                        void* workspace, size_t workspace_bytes, hipStream_t stream) {
    const float alpha = 1.0f, beta = 0.0f;
    return library().matmul(ctx.handle, plan.op, &alpha, b, plan.b_layout, a, plan.a_layout, &beta, c,
                            plan.c_layout, c, plan.c_layout, &plan.algo, workspace, workspace_bytes, stream);
}

// Builds the descriptors of (m, n, k), asks the library for up to 32
// algorithms that fit the workspace, times each once after a warm-up launch
// on the caller's stream, and keeps the fastest.
int make_plan(Context& ctx, uint64_t m, uint64_t n, uint64_t k, const void* a, const void* b, void* c,
              void* workspace, size_t workspace_bytes, hipStream_t stream, std::unique_ptr<Plan>& out) {
    const Library& l = library();
    auto plan = std::make_unique<Plan>();
    hipblasStatus_t st = l.desc_create(&plan->op, HIPBLAS_COMPUTE_32F, HIP_R_32F);
    if (st != HIPBLAS_STATUS_SUCCESS) return ctx.fail_blas(st, "hipblasLtMatmulDescCreate");
    st = l.layout_create(&plan->b_layout, HIP_R_16F, n, k, static_cast<int64_t>(n));
    if (st != HIPBLAS_STATUS_SUCCESS) return ctx.fail_blas(st, "hipblasLtMatrixLayoutCreate(B)");
    st = l.layout_create(&plan->a_layout, HIP_R_16F, k, m, static_cast<int64_t>(k));
    if (st != HIPBLAS_STATUS_SUCCESS) return ctx.fail_blas(st, "hipblasLtMatrixLayoutCreate(A)");
    st = l.layout_create(&plan->c_layout, HIP_R_32F, n, m, static_cast<int64_t>(n));
    if (st != HIPBLAS_STATUS_SUCCESS) return ctx.fail_blas(st, "hipblasLtMatrixLayoutCreate(C)");

    hipblasLtMatmulPreference_t pref = nullptr;
    st = l.pref_create(&pref);
    if (st != HIPBLAS_STATUS_SUCCESS) return ctx.fail_blas(st, "hipblasLtMatmulPreferenceCreate");
    const uint64_t limit = workspace_bytes;
    st = l.pref_set(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &limit, sizeof(limit));
    hipblasLtMatmulHeuristicResult_t found[kCandidates]{};
    int count = 0;
    if (st == HIPBLAS_STATUS_SUCCESS)
        st = l.heuristic(ctx.handle, plan->op, plan->b_layout, plan->a_layout, plan->c_layout, plan->c_layout,
                         pref, kCandidates, found, &count);
    l.pref_destroy(pref);
    if (st != HIPBLAS_STATUS_SUCCESS) return ctx.fail_blas(st, "hipblasLtMatmulAlgoGetHeuristic");
    if (count <= 0) return ctx.fail(kArgumentError, "hipBLASLt offers no algorithm for this shape");

    hipEvent_t start = nullptr, stop = nullptr;
    hipError_t he = hipEventCreate(&start);
    if (he != hipSuccess) return ctx.fail_hip(he, "hipEventCreate");
    he = hipEventCreate(&stop);
    if (he != hipSuccess) {
        (void)hipEventDestroy(start);
        return ctx.fail_hip(he, "hipEventCreate");
    }
    float best = std::numeric_limits<float>::infinity();
    hipblasLtMatmulAlgo_t best_algo{};
    for (int i = 0; i < count; ++i) {
        if (found[i].state != HIPBLAS_STATUS_SUCCESS || found[i].workspaceSize > workspace_bytes) continue;
        plan->algo = found[i].algo;
        if (enqueue(ctx, *plan, a, b, c, workspace, workspace_bytes, stream) != HIPBLAS_STATUS_SUCCESS) continue;
        float ms = 0.0f;
        if (hipEventRecord(start, stream) != hipSuccess ||
            enqueue(ctx, *plan, a, b, c, workspace, workspace_bytes, stream) != HIPBLAS_STATUS_SUCCESS ||
            hipEventRecord(stop, stream) != hipSuccess || hipEventSynchronize(stop) != hipSuccess ||
            hipEventElapsedTime(&ms, start, stop) != hipSuccess)
            continue;
        if (ms < best) {
            best = ms;
            best_algo = found[i].algo;
        }
    }
    (void)hipEventDestroy(start);
    (void)hipEventDestroy(stop);
    if (!std::isfinite(best)) return ctx.fail(kArgumentError, "no hipBLASLt algorithm launched for this shape");
    plan->algo = best_algo;
    out = std::move(plan);
    return 0;
}

// Output of an empty sum (k == 0): zeros, written by a kernel rather than
// hipMemsetAsync so the call can be captured in a graph.
__global__ void zero_f32(float* __restrict__ c, uint64_t count) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < count) c[i] = 0.0f;
}

}  // namespace
}  // namespace mote::dense

using mote::dense::Context;

MOTE_EXPORT int mote_hipblaslt_create(void** output) noexcept {
    if (output == nullptr) return mote::dense::kArgumentError;
    *output = nullptr;
    const auto& lib = mote::dense::library();
    if (!lib.error.empty()) return mote::dense::kArgumentError;
    try {
        auto ctx = std::make_unique<Context>();
        const hipblasStatus_t st = lib.create(&ctx->handle);
        if (st != HIPBLAS_STATUS_SUCCESS) return static_cast<int>(st);
        *output = ctx.release();
        return 0;
    } catch (...) {
        return mote::dense::kArgumentError;
    }
}

MOTE_EXPORT void mote_hipblaslt_destroy(void* handle) noexcept { delete static_cast<Context*>(handle); }

MOTE_EXPORT const char* mote_hipblaslt_last_error(void* handle) noexcept {
    const auto* ctx = static_cast<const Context*>(handle);
    return ctx == nullptr ? nullptr : ctx->last_error.c_str();
}

MOTE_EXPORT int mote_hipblaslt_matmul_f16_f32(void* handle, uint64_t m, uint64_t n, uint64_t k, const void* lhs,
                                              const void* rhs, void* output, void* workspace,
                                              size_t workspace_bytes, void* stream) noexcept {
    auto* ctx = static_cast<Context*>(handle);
    if (ctx == nullptr) return mote::dense::kArgumentError;
    std::lock_guard<std::mutex> lock(ctx->mutex);
    if (lhs == nullptr || rhs == nullptr || output == nullptr || workspace == nullptr || stream == nullptr)
        return ctx->fail(mote::dense::kArgumentError, "hipBLASLt matmul received a null pointer");
    const auto s = static_cast<hipStream_t>(stream);
    if (m == 0 || n == 0) {  // nothing to write
        ctx->last_error.clear();
        return 0;
    }
    if (k == 0) {
        const uint64_t count = m * n;
        if (count / m != n || count > (uint64_t{1} << 40))
            return ctx->fail(mote::dense::kArgumentError, "hipBLASLt matmul output too large");
        hipLaunchKernelGGL(mote::dense::zero_f32, dim3(static_cast<uint32_t>((count + 255) / 256)), dim3(256), 0, s,
                           static_cast<float*>(output), count);
        const hipError_t he = hipGetLastError();
        if (he != hipSuccess) return ctx->fail_hip(he, "zero fill");
        ctx->last_error.clear();
        return 0;
    }
    try {
        const auto key = std::make_tuple(m, n, k);
        auto it = ctx->plans.find(key);
        if (it == ctx->plans.end()) {
            std::unique_ptr<mote::dense::Plan> plan;
            const int status =
                mote::dense::make_plan(*ctx, m, n, k, lhs, rhs, output, workspace, workspace_bytes, s, plan);
            if (status != 0) return status;
            it = ctx->plans.emplace(key, std::move(plan)).first;
        }
        const hipblasStatus_t st =
            mote::dense::enqueue(*ctx, *it->second, lhs, rhs, output, workspace, workspace_bytes, s);
        if (st != HIPBLAS_STATUS_SUCCESS) return ctx->fail_blas(st, "hipblasLtMatmul");
        ctx->last_error.clear();
        return 0;
    } catch (const std::exception& e) {
        return ctx->fail(mote::dense::kArgumentError, e.what());
    } catch (...) {
        return ctx->fail(mote::dense::kArgumentError, "unknown C++ exception");
    }
}

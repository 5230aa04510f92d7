// abi_internal.h -- what the C-ABI translation units (qmm_abi.cpp,
// llama.cpp) share: the context and weight objects behind the opaque
// handles of include/rce_qmm.h, the thread-local last-error text and the
// device-memory helpers.  Not installed.
#pragma once

#include "../../include/rce_qmm.h"
#include "qmm_internal.h"

#include <algorithm>
#include <atomic>
#include <memory>
#include <string>
#include <vector>

namespace rce_qmm_abi {

using namespace rce_qmm;

// Record `msg` as this thread's last error (rce_qmm_last_error) and return s.
rce_qmm_status fail(rce_qmm_status s, const std::string &msg);

inline rce_qmm_status hip_fail(hipError_t e, const char *what) {
    return fail(RCE_QMM_HIP_ERROR, std::string(what) + ": " + hipGetErrorString(e));
}

#define HIP_TRY(expr)                                       \
    do {                                                    \
        hipError_t e_ = (expr);                             \
        if (e_ != hipSuccess) return hip_fail(e_, #expr);   \
    } while (0)

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// A device allocation shared by a weight and its views.
struct DevAlloc {
    void *p = nullptr;
    int device = 0;
    ~DevAlloc() {
        if (p) {
            int cur = 0;
            (void)hipGetDevice(&cur);
            (void)hipSetDevice(device);
            (void)hipFree(p);
            (void)hipSetDevice(cur);
        }
    }
};

// Grow-only device buffer owned by a context.
struct Scratch {
    void *p = nullptr;
    size_t cap = 0;
};

}  // namespace rce_qmm_abi

struct rce_qmm_context {
    int device = 0;
    hipStream_t stream = nullptr;
    // Holders: the caller (until rce_qmm_context_destroy) and every decoder
    // made on the context (until rce_qmm_llama_destroy); the last release
    // frees it, so a decoder destroyed after its context stays valid.
    std::atomic<int> refs{1};
    rce_qmm_abi::Scratch a_in, a_f32, out;
    rce_qmm_abi::Scratch a_f16;  // f32 activations rounded to f16 for the MFMA GEMM
    rce_qmm_abi::Scratch act_q;  // several tokens' Q8 activations, quantized once per launch
    // grouped experts: grouping metadata, expert tables, stage buffers
    rce_qmm_abi::Scratch moe_meta, moe_wtab, moe_x, moe_h, moe_h16, moe_y, moe_u;
    std::vector<rce_qmm::DevWeight> moe_wtab_host;  // what moe_wtab holds
};

struct rce_qmm_weight {
    std::shared_ptr<rce_qmm_abi::DevAlloc> alloc;
    rce_qmm::DevWeight dw{};
    size_t host_row_bytes = 0;  // GGUF bytes per row
    size_t len = 0;             // GGUF byte length of this view
    int device = 0;
};

namespace rce_qmm_abi {

// Drop one holder of the context (see rce_qmm_context::refs).
void context_release(rce_qmm_context *ctx);

inline rce_qmm_status set_device(int dev) {
    HIP_TRY(hipSetDevice(dev));
    return RCE_QMM_OK;
}

// Make `s` hold at least `bytes`; waits for the context's stream before a
// reallocation so in-flight kernels never see a freed buffer.
inline rce_qmm_status ensure(rce_qmm_context *ctx, Scratch &s, size_t bytes, hipStream_t other) {
    if (s.cap >= bytes) return RCE_QMM_OK;
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    if (other && other != ctx->stream) HIP_TRY(hipStreamSynchronize(other));
    if (s.p) HIP_TRY(hipFree(s.p));
    s.p = nullptr;
    s.cap = 0;
    size_t cap = align_up(std::max<size_t>(bytes, 4096), 4096);
    hipError_t e = hipMalloc(&s.p, cap);
    if (e != hipSuccess) return fail(RCE_QMM_OUT_OF_MEMORY, std::string("scratch hipMalloc: ") + hipGetErrorString(e));
    s.cap = cap;
    return RCE_QMM_OK;
}

// mm_batched_dev's device-side core (qmm_abi.cpp).  fixed == nullptr: the
// scratch comes from the context's grow-only buffers; else from the
// fixed_cap bytes at `fixed`, with no allocation (RCE_QMM_BAD_SHAPE when
// the call needs more than batched_scratch_bytes allows).
rce_qmm_status run_batched(rce_qmm_context *ctx, const void *a_dev, uint32_t a_dtype, size_t t_rows,
                           const rce_qmm_weight *w, float *out_dev, rce_qmm_mode mode, hipStream_t s, void *fixed,
                           size_t fixed_cap);
// Scratch bytes run_batched needs for these arguments.
size_t batched_scratch_bytes(const DevWeight &dw, uint32_t a_dtype, size_t t_rows, rce_qmm_mode mode);
// Resolve the device address of the no-allocation entry point's fixed
// scratch on `device` (the current device), once per device (noalloc.hip).
rce_qmm_status noalloc_setup(int device);

inline rce_qmm_status check_weight_ctx(rce_qmm_context *ctx, const rce_qmm_weight *w) {
    if (!ctx || !w) return fail(RCE_QMM_NULL_ARGUMENT, "null context or weight");
    if (ctx->device != w->device) return fail(RCE_QMM_BAD_SHAPE, "weight lives on another device than the context");
    return RCE_QMM_OK;
}

}  // namespace rce_qmm_abi

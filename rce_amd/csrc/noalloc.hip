// noalloc.hip -- rce_qmm_mm_batched_dev_noalloc: mm_batched_dev for callers
// that cannot allocate device memory (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc).  It runs the same kernels
// as rce_qmm_mm_batched_dev; the scratch those need (F16 activations widened
// to f32, several tokens' Q8 activations quantized once, F32 activations
// rounded to f16 for the MFMA GEMM) lives in `scratch`, a fixed device array
// that every GPU the library runs on holds until the process ends.
//
// In host code `scratch` names a host-side stand-in, not device memory: the
// array's device address on each GPU is resolved once, with that GPU
// current, by hipGetSymbolAddress (noalloc_setup, called by
// rce_qmm_context_create) and only that address is handed to kernels.
// Every call on one GPU shares the array and it keeps the last call's
// contents; nothing in it needs to start at zero (each call writes every
// byte it reads).  Calls that overlap on one GPU race.
#include "abi_internal.h"

#include <mutex>
#include <string>

static __device__ __align__(256) unsigned char scratch[RCE_QMM_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 256;
std::mutex g_mu;
void *g_ptr[MAX_DEVICES];  // the device address of `scratch` on each GPU (null until resolved)

}  // namespace

rce_qmm_status rce_qmm_abi::noalloc_setup(int device) {
    if (device < 0 || device >= MAX_DEVICES) return fail(RCE_QMM_NO_DEVICE, "device index beyond the library's table");
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_ptr[device]) return RCE_QMM_OK;
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
    g_ptr[device] = p;
    return RCE_QMM_OK;
}

extern "C" rce_qmm_status rce_qmm_mm_batched_dev_noalloc(rce_qmm_context *ctx, const void *a_dev, uint32_t a_dtype,
                                                         size_t t_rows, const rce_qmm_weight *w, float *out_dev,
                                                         rce_qmm_mode mode, void *stream) {
    using namespace rce_qmm_abi;
    rce_qmm_status st = check_weight_ctx(ctx, w);
    if (st) return st;
    if ((!a_dev || !out_dev) && t_rows) return fail(RCE_QMM_NULL_ARGUMENT, "null device buffer");
    void *p = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        p = ctx->device >= 0 && ctx->device < MAX_DEVICES ? g_ptr[ctx->device] : nullptr;
    }
    if (!p) return fail(RCE_QMM_INTERNAL, "the fixed scratch of device " + std::to_string(ctx->device) + " was not resolved");
    if ((st = set_device(ctx->device))) return st;
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
    return run_batched(ctx, a_dev, a_dtype, t_rows, w, out_dev, mode, s, p, RCE_QMM_NOALLOC_SCRATCH_BYTES);
}

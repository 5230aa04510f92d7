// qmm_abi.cpp -- the extern "C" boundary of librce_qmm.so (include/rce_qmm.h).
//
// Owns device memory and streams: a context is one device + one HIP stream +
// scratch; a weight is a device-resident copy of GGUF bytes in the layout
// its kernels read (same byte count), shared by its sub-views.  No C++
// exception crosses the ABI; failures set a thread-local message
// (rce_qmm_last_error), the convention of compute/crates/rce-c/include/rce.h.
#include "abi_internal.h"
#include "lds_limit.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <vector>

using namespace rce_qmm;

namespace rce_qmm_abi {

thread_local std::string g_last_error;

rce_qmm_status fail(rce_qmm_status s, const std::string &msg) {
    g_last_error = msg;
    return s;
}

}  // namespace rce_qmm_abi

using namespace rce_qmm_abi;

namespace {

bool block_geometry(uint32_t t, size_t &qk, size_t &bb) {
    switch (t) {
    case T_F32: qk = 1; bb = 4; return true;
    case T_F16: case T_BF16: qk = 1; bb = 2; return true;
    case T_Q4_0: qk = 32; bb = 18; return true;
    case T_Q4_1: qk = 32; bb = 20; return true;
    case T_Q5_0: qk = 32; bb = 22; return true;
    case T_Q8_0: qk = 32; bb = 34; return true;
    case T_Q3_K: qk = 256; bb = 110; return true;
    case T_Q4_K: qk = 256; bb = 144; return true;
    case T_Q5_K: qk = 256; bb = 176; return true;
    case T_Q6_K: qk = 256; bb = 210; return true;
    case T_I2_S: qk = 128; bb = 32; return true;  // plus the tensor's f32 scale
    case T_Q1_0: qk = 128; bb = 18; return true;
    case T_Q2_0: qk = 128; bb = 34; return true;
    case T_STQ1_0: qk = 256; bb = 42; return true;
    default: return false;
    }
}

// Every kernel family: decode kernels (EXACT, Q8) and the MFMA GEMM.
bool supports_mode(uint32_t dtype, size_t n_cols, int mode) {
    if (mode == RCE_QMM_MODE_F16_MFMA) return gemm_supports(dtype, n_cols) || gemm_gen_supports(dtype, n_cols);
    return gpu_supports(dtype, n_cols, mode);
}

// Scratch pointers of one mm_batched_dev call: each is null when the
// call's (a_dtype, mode, shape) does not need it.
struct BatchedScratch {
    float *a_f32 = nullptr;       // F16 activations widened to f32 (EXACT, Q8)
    unsigned char *act_q = nullptr;  // Q8 activations of several tokens, quantized once
    void *a_f16 = nullptr;        // F32 activations rounded to f16 (F16_MFMA)
};

}  // namespace

// The scratch bytes mm_batched_dev needs for these arguments (the parts
// BatchedScratch names, each rounded up to 256 bytes), given a supported
// (dtype, n_cols, mode).
size_t rce_qmm_abi::batched_scratch_bytes(const DevWeight &dw, uint32_t a_dtype, size_t t_rows, rce_qmm_mode mode) {
    const size_t k = dw.n_cols;
    if (t_rows == 0 || dw.n_rows == 0) return 0;
    if (mode == RCE_QMM_MODE_F16_MFMA) return a_dtype == T_F16 ? 0 : align_up(t_rows * k * 2, 256);
    size_t b = 0;
    if (a_dtype == T_F16) b += align_up(t_rows * k * sizeof(float), 256);
    if (mode == RCE_QMM_MODE_Q8 && gemv_q8_pre_supports(dw.dtype, k, t_rows)) b += align_up(t_rows * (k + k / 8 + k / 4), 256);
    return b;
}

namespace {

// The prefill GEMM; f32 activations are rounded to f16 first (into sc.a_f16).
rce_qmm_status run_gemm(const void *a_dev, bool a_f16, size_t t_rows, const DevWeight &dw, float *out_dev,
                        const BatchedScratch &sc, hipStream_t s) {
    const void *a = a_dev;
    if (!a_f16) {
        HIP_TRY(launch_f32_to_f16(static_cast<const float *>(a_dev), sc.a_f16, t_rows * dw.n_cols, s));
        a = sc.a_f16;
    }
    if (reinterpret_cast<uintptr_t>(a) % 16)
        return fail(RCE_QMM_BAD_SHAPE, "F16 activations of the F16_MFMA GEMM must be 16-byte aligned");
    if (gemm_supports(dw.dtype, dw.n_cols) || gemm_q8_supports(dw.dtype, dw.n_cols)) {
        // The kernel's activation offsets are 32-bit: slices of whole
        // 128-row tiles below 2^32 bytes each (each output's sum does not
        // depend on the slicing).
        const size_t k = dw.n_cols, max_rows = ((((size_t)1 << 32) - 1) / (k * 2)) / 128 * 128;
        if (max_rows == 0)
            return fail(RCE_QMM_BAD_SHAPE, "n_cols " + std::to_string(k) + " is too long for the F16_MFMA GEMM");
        const _Float16 *a16 = static_cast<const _Float16 *>(a);
        for (size_t r0 = 0; r0 < t_rows; r0 += max_rows) {
            const size_t rows = t_rows - r0 < max_rows ? t_rows - r0 : max_rows;
            HIP_TRY(launch_gemm_f16(dw, a16 + r0 * k, rows, out_dev + r0 * dw.n_rows, s));
        }
    } else {
        HIP_TRY(launch_gemm_gen(dw, a, t_rows, out_dev, s));
    }
    return RCE_QMM_OK;
}

}  // namespace

// Device-side core shared by the host and device entry points.  fixed ==
// nullptr: the scratch comes from the context's grow-only buffers (which
// may allocate); else from the fixed_cap bytes at fixed (no allocation;
// RCE_QMM_BAD_SHAPE when the call needs more).
rce_qmm_status rce_qmm_abi::run_batched(rce_qmm_context *ctx, const void *a_dev, uint32_t a_dtype, size_t t_rows,
                                        const rce_qmm_weight *w, float *out_dev, rce_qmm_mode mode, hipStream_t s,
                                        void *fixed, size_t fixed_cap) {
    const DevWeight &dw = w->dw;
    if (!supports_mode(dw.dtype, dw.n_cols, (int)mode))
        return fail(RCE_QMM_UNSUPPORTED_DTYPE, "dtype " + std::to_string(dw.dtype) + " with n_cols " +
                                                   std::to_string(dw.n_cols) + " has no GPU kernel in mode " +
                                                   std::to_string((int)mode));
    if (a_dtype != T_F32 && a_dtype != T_F16) return fail(RCE_QMM_UNSUPPORTED_DTYPE, "activations must be F32 or F16");
    if (mode != RCE_QMM_MODE_EXACT && mode != RCE_QMM_MODE_Q8 && mode != RCE_QMM_MODE_F16_MFMA)
        return fail(RCE_QMM_BAD_SHAPE, "unknown mode");
    if (t_rows == 0 || dw.n_rows == 0) return RCE_QMM_OK;
    const size_t k = dw.n_cols;
    const bool mfma = mode == RCE_QMM_MODE_F16_MFMA;
    const bool widen = !mfma && a_dtype == T_F16;
    const bool preq = mode == RCE_QMM_MODE_Q8 && gemv_q8_pre_supports(dw.dtype, k, t_rows);
    const size_t f32_b = widen ? t_rows * k * sizeof(float) : 0;
    const size_t q8_b = preq ? t_rows * (k + k / 8 + k / 4) : 0;  // xq, dx, s16
    const size_t f16_b = mfma && a_dtype == T_F32 ? t_rows * k * 2 : 0;
    BatchedScratch sc;
    rce_qmm_status st;
    if (fixed) {
        const size_t need = batched_scratch_bytes(dw, a_dtype, t_rows, mode);
        if (need > fixed_cap)
            return fail(RCE_QMM_BAD_SHAPE, "the call needs " + std::to_string(need) + " bytes of scratch; the fixed scratch holds " +
                                               std::to_string(fixed_cap));
        unsigned char *p = static_cast<unsigned char *>(fixed);
        if (f32_b) { sc.a_f32 = reinterpret_cast<float *>(p); p += align_up(f32_b, 256); }
        if (q8_b) { sc.act_q = p; p += align_up(q8_b, 256); }
        if (f16_b) { sc.a_f16 = p; p += align_up(f16_b, 256); }
    } else {
        if (f32_b) {
            if ((st = ensure(ctx, ctx->a_f32, f32_b, s))) return st;
            sc.a_f32 = static_cast<float *>(ctx->a_f32.p);
        }
        if (q8_b) {
            if ((st = ensure(ctx, ctx->act_q, q8_b, s))) return st;
            sc.act_q = static_cast<unsigned char *>(ctx->act_q.p);
        }
        if (f16_b) {
            if ((st = ensure(ctx, ctx->a_f16, f16_b, s))) return st;
            sc.a_f16 = ctx->a_f16.p;
        }
    }
    if (mfma) return run_gemm(a_dev, a_dtype == T_F16, t_rows, dw, out_dev, sc, s);
    const float *a32 = static_cast<const float *>(a_dev);
    if (widen) {
        HIP_TRY(launch_f16_to_f32(static_cast<const uint16_t *>(a_dev), sc.a_f32, t_rows * k, s));
        a32 = sc.a_f32;
    }
    if (preq) {
        HIP_TRY(launch_gemv_q8_pre(dw, a32, t_rows, out_dev, sc.act_q, s));
        return RCE_QMM_OK;
    }
    HIP_TRY(launch_gemv(dw, a32, t_rows, out_dev, (int)mode, s));
    return RCE_QMM_OK;
}

namespace {

rce_qmm_status host_batched(rce_qmm_context *ctx, const float *a, size_t t_rows, const rce_qmm_weight *w,
                            float *out) {
    rce_qmm_status st = check_weight_ctx(ctx, w);
    if (st) return st;
    if (!a || !out) return fail(RCE_QMM_NULL_ARGUMENT, "null activation or output");
    if ((st = set_device(ctx->device))) return st;
    const DevWeight &dw = w->dw;
    if (!gpu_supports(dw.dtype, dw.n_cols, RCE_QMM_MODE_EXACT))
        return fail(RCE_QMM_UNSUPPORTED_DTYPE, "dtype " + std::to_string(dw.dtype) + " with n_cols " +
                                                   std::to_string(dw.n_cols) + " has no GPU kernel");
    if (t_rows == 0 || dw.n_rows == 0) return RCE_QMM_OK;
    const size_t abytes = t_rows * dw.n_cols * sizeof(float), obytes = t_rows * dw.n_rows * sizeof(float);
    if ((st = ensure(ctx, ctx->a_in, abytes, nullptr))) return st;
    if ((st = ensure(ctx, ctx->out, obytes, nullptr))) return st;
    HIP_TRY(hipMemcpyAsync(ctx->a_in.p, a, abytes, hipMemcpyHostToDevice, ctx->stream));
    if ((st = run_batched(ctx, ctx->a_in.p, T_F32, t_rows, w, static_cast<float *>(ctx->out.p), RCE_QMM_MODE_EXACT,
                          ctx->stream, nullptr, 0)))
        return st;
    HIP_TRY(hipMemcpyAsync(out, ctx->out.p, obytes, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return RCE_QMM_OK;
}

}  // namespace

extern "C" {

const char *rce_qmm_last_error(void) { return g_last_error.c_str(); }

const char *rce_qmm_status_str(rce_qmm_status s) {
    switch (s) {
    case RCE_QMM_OK: return "ok";
    case RCE_QMM_NULL_ARGUMENT: return "null argument";
    case RCE_QMM_BAD_SHAPE: return "bad shape";
    case RCE_QMM_UNSUPPORTED_DTYPE: return "unsupported dtype";
    case RCE_QMM_NO_DEVICE: return "no device";
    case RCE_QMM_HIP_ERROR: return "hip error";
    case RCE_QMM_OUT_OF_MEMORY: return "out of memory";
    case RCE_QMM_INTERNAL: return "internal error";
    case RCE_QMM_NOT_FOUND: return "not found";
    case RCE_QMM_PARSE_ERROR: return "parse error";
    case RCE_QMM_IO_ERROR: return "i/o error";
    }
    return "unknown status";
}

uint32_t rce_qmm_abi_version(void) { return RCE_QMM_ABI_VERSION; }

rce_qmm_status rce_qmm_context_create(int device, rce_qmm_context **out) {
    if (!out) return fail(RCE_QMM_NULL_ARGUMENT, "null out");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) return fail(RCE_QMM_NO_DEVICE, "no HIP device");
    if (device < 0 || device >= n) return fail(RCE_QMM_NO_DEVICE, "device index out of range");
    HIP_TRY(hipSetDevice(device));
    rce_qmm_status st = noalloc_setup(device);
    if (st) return st;
    HIP_TRY(rce_qmm::chain_prepare_lds());
    HIP_TRY(rce_qmm::q6_prepare_lds());
    HIP_TRY(rce_qmm::gemm_prepare_lds());
    hipStream_t s = nullptr;
    HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    rce_qmm_context *c = new (std::nothrow) rce_qmm_context();
    if (!c) {
        (void)hipStreamDestroy(s);
        return fail(RCE_QMM_OUT_OF_MEMORY, "context allocation");
    }
    c->device = device;
    c->stream = s;
    *out = c;
    return RCE_QMM_OK;
}

void rce_qmm_context_destroy(rce_qmm_context *ctx) {
    if (ctx) context_release(ctx);
}

}  // extern "C"

void rce_qmm_abi::context_release(rce_qmm_context *ctx) {
    if (ctx->refs.fetch_sub(1) != 1) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (Scratch *s : {&ctx->a_in, &ctx->a_f32, &ctx->out, &ctx->a_f16, &ctx->act_q, &ctx->moe_meta, &ctx->moe_wtab, &ctx->moe_x,
                       &ctx->moe_h, &ctx->moe_h16, &ctx->moe_y, &ctx->moe_u})
        if (s->p) (void)hipFree(s->p);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

extern "C" {

rce_qmm_status rce_qmm_context_stream(rce_qmm_context *ctx, void **stream) {
    if (!ctx || !stream) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    *stream = ctx->stream;
    return RCE_QMM_OK;
}

rce_qmm_status rce_qmm_synchronize(rce_qmm_context *ctx) {
    if (!ctx) return fail(RCE_QMM_NULL_ARGUMENT, "null context");
    HIP_TRY(hipSetDevice(ctx->device));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return RCE_QMM_OK;
}

int rce_qmm_supports(uint32_t dtype, size_t n_cols, rce_qmm_mode mode) {
    return supports_mode(dtype, n_cols, (int)mode) ? 1 : 0;
}

rce_qmm_status rce_qmm_weight_from_bytes(rce_qmm_context *ctx, uint32_t dtype, size_t n_rows, size_t n_cols,
                                         const uint8_t *bytes, size_t len, rce_qmm_weight **out) {
    if (!ctx || !out || (!bytes && len)) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    *out = nullptr;
    size_t qk, bb;
    if (!block_geometry(dtype, qk, bb)) return fail(RCE_QMM_UNSUPPORTED_DTYPE, "unknown dtype " + std::to_string(dtype));
    if (n_cols == 0 || n_cols % qk)
        return fail(RCE_QMM_BAD_SHAPE, "n_cols " + std::to_string(n_cols) + " is not a multiple of the block size " +
                                           std::to_string(qk));
    const size_t rowb = n_cols / qk * bb;
    size_t want_len = 0;
    if (__builtin_mul_overflow(n_rows, rowb, &want_len) ||
        __builtin_add_overflow(want_len, (size_t)(dtype == T_I2_S ? 4 : 0), &want_len))  // I2_S: codes, then one f32 scale
        return fail(RCE_QMM_BAD_SHAPE, "n_rows * row_bytes overflows size_t");
    if (want_len > ((size_t)1 << 48))  // the device layout adds padding per row: keep its size far from wrapping
        return fail(RCE_QMM_BAD_SHAPE, "weights larger than 2^48 bytes");
    if (len != want_len)
        return fail(RCE_QMM_BAD_SHAPE, "len " + std::to_string(len) + " != " + std::to_string(want_len) +
                                           (dtype == T_I2_S ? " (n_rows*row_bytes + the f32 scale)" : " (n_rows*row_bytes)"));
    if (!gpu_supports(dtype, n_cols, RCE_QMM_MODE_EXACT))
        return fail(RCE_QMM_UNSUPPORTED_DTYPE, "dtype " + std::to_string(dtype) + " with n_cols " + std::to_string(n_cols) +
                                                   " has no GPU kernel");
    rce_qmm_status st = set_device(ctx->device);
    if (st) return st;

    DevWeight dw{};
    dw.dtype = dtype;
    dw.n_rows = n_rows;
    dw.n_cols = n_cols;
    const size_t total = plan_layout(dw);
    std::vector<uint8_t> host;
    try {
        host.assign(std::max<size_t>(total, 1), 0);
    } catch (...) {
        return fail(RCE_QMM_OUT_OF_MEMORY, "host staging for relayout");
    }
    relayout_host(bytes, dw, host.data());
    auto alloc = std::make_shared<DevAlloc>();
    alloc->device = ctx->device;
    const size_t pad = layout_pad_bytes(dw);  // rows a decode tile may read past the end (never folded)
    hipError_t e = hipMalloc(&alloc->p, std::max<size_t>(total + pad, 256));
    if (e != hipSuccess) {
        alloc->p = nullptr;
        return fail(RCE_QMM_OUT_OF_MEMORY, std::string("weight hipMalloc: ") + hipGetErrorString(e));
    }
    HIP_TRY(hipMemcpyAsync(alloc->p, host.data(), total, hipMemcpyHostToDevice, ctx->stream));
    if (pad) HIP_TRY(hipMemsetAsync(static_cast<uint8_t *>(alloc->p) + total, 0, pad, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    dw.base = static_cast<const uint8_t *>(alloc->p);
    if (dtype == T_I2_S) dw.aux = dw.base + dw.plane1;
    rce_qmm_weight *w = new (std::nothrow) rce_qmm_weight();
    if (!w) return fail(RCE_QMM_OUT_OF_MEMORY, "weight handle");
    w->alloc = alloc;
    w->dw = dw;
    w->host_row_bytes = rowb;
    w->len = len;
    w->device = ctx->device;
    *out = w;
    return RCE_QMM_OK;
}

rce_qmm_status rce_qmm_weight_sub_view(const rce_qmm_weight *w, size_t byte_offset, size_t byte_len, size_t n_rows,
                                       size_t n_cols, rce_qmm_weight **out) {
    if (!w || !out) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    *out = nullptr;
    if (byte_offset > w->len || byte_len > w->len - byte_offset)
        return fail(RCE_QMM_BAD_SHAPE, "sub_view out of bounds: " + std::to_string(byte_offset) + "+" +
                                           std::to_string(byte_len) + " > " + std::to_string(w->len));
    if (n_cols != w->dw.n_cols) return fail(RCE_QMM_BAD_SHAPE, "sub_view must keep n_cols");
    const size_t rb = w->host_row_bytes;
    size_t view_bytes = 0;
    if (rb == 0 || byte_offset % rb || __builtin_mul_overflow(n_rows, rb, &view_bytes) || byte_len != view_bytes)
        return fail(RCE_QMM_BAD_SHAPE, "sub_view must cover whole rows of the parent");
    const size_t row0 = byte_offset / rb;
    if (w->dw.dtype == T_I2_S)  // one scale per tensor, after all rows
        return fail(RCE_QMM_BAD_SHAPE, "I2_S has one scale per tensor: no sub_view");
    DevWeight dw = w->dw;
    dw.n_rows = n_rows;
    if (dw.layout == LAYOUT_IL64_Q6_K || dw.layout == LAYOUT_IL64_ROWS) {
        if (row0 % 64) return fail(RCE_QMM_BAD_SHAPE, "Q6_K / F32 / F16 / BF16 sub_view must start on a multiple of 64 rows");
        dw.base += (row0 / 64) * dw.group_stride;
    } else {
        dw.base += row0 * dw.row_stride;
    }
    rce_qmm_weight *v = new (std::nothrow) rce_qmm_weight();
    if (!v) return fail(RCE_QMM_OUT_OF_MEMORY, "weight handle");
    v->alloc = w->alloc;
    v->dw = dw;
    v->host_row_bytes = rb;
    v->len = byte_len;
    v->device = w->device;
    *out = v;
    return RCE_QMM_OK;
}

void rce_qmm_weight_destroy(rce_qmm_weight *w) { delete w; }

rce_qmm_status rce_qmm_weight_info(const rce_qmm_weight *w, uint32_t *dtype, size_t *n_rows, size_t *n_cols,
                                   size_t *len) {
    if (!w) return fail(RCE_QMM_NULL_ARGUMENT, "null weight");
    if (dtype) *dtype = w->dw.dtype;
    if (n_rows) *n_rows = w->dw.n_rows;
    if (n_cols) *n_cols = w->dw.n_cols;
    if (len) *len = w->len;
    return RCE_QMM_OK;
}

rce_qmm_status rce_qmm_mm_1d(rce_qmm_context *ctx, const float *a, const rce_qmm_weight *w, float *out) {
    return host_batched(ctx, a, 1, w, out);
}

rce_qmm_status rce_qmm_mm_1d_serial(rce_qmm_context *ctx, const float *a, const rce_qmm_weight *w, float *out) {
    return host_batched(ctx, a, 1, w, out);
}

rce_qmm_status rce_qmm_mm_batched(rce_qmm_context *ctx, const float *a, size_t t_rows, const rce_qmm_weight *w,
                                  float *out) {
    return host_batched(ctx, a, t_rows, w, out);
}

rce_qmm_status rce_qmm_dequant_row(rce_qmm_context *ctx, const rce_qmm_weight *w, size_t row, float *out) {
    rce_qmm_status st = check_weight_ctx(ctx, w);
    if (st) return st;
    if (!out) return fail(RCE_QMM_NULL_ARGUMENT, "null output");
    if (row >= w->dw.n_rows) return fail(RCE_QMM_BAD_SHAPE, "row out of range");
    if ((st = set_device(ctx->device))) return st;
    const size_t bytes = w->dw.n_cols * sizeof(float);
    if ((st = ensure(ctx, ctx->out, bytes, nullptr))) return st;
    HIP_TRY(launch_dequant_row(w->dw, row, static_cast<float *>(ctx->out.p), ctx->stream));
    HIP_TRY(hipMemcpyAsync(out, ctx->out.p, bytes, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return RCE_QMM_OK;
}

rce_qmm_status rce_qmm_mm_batched_dev(rce_qmm_context *ctx, const void *a_dev, uint32_t a_dtype, size_t t_rows,
                                      const rce_qmm_weight *w, float *out_dev, rce_qmm_mode mode, void *stream) {
    rce_qmm_status st = check_weight_ctx(ctx, w);
    if (st) return st;
    if ((!a_dev || !out_dev) && t_rows) return fail(RCE_QMM_NULL_ARGUMENT, "null device buffer");
    if ((st = set_device(ctx->device))) return st;
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
    return run_batched(ctx, a_dev, a_dtype, t_rows, w, out_dev, mode, s, nullptr, 0);
}

rce_qmm_status rce_qmm_moe_router(const float *logits, size_t n_tokens, size_t n_expert, size_t top_k,
                                  int normalize, int32_t *ids, float *weights) {
    if (!logits || !ids || !weights) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    if (n_expert == 0 || top_k == 0 || top_k > n_expert) return fail(RCE_QMM_BAD_SHAPE, "need 0 < top_k <= n_expert");
    std::vector<float> probs(n_expert);
    std::vector<int32_t> order(n_expert);
    for (size_t t = 0; t < n_tokens; t++) {
        const float *l = logits + t * n_expert;
        // rce-op-moe/src/lib.rs L50-55: max-subtracted softmax over all experts.
        float mx = -INFINITY;
        for (size_t e = 0; e < n_expert; e++) mx = std::fmax(mx, l[e]);
        for (size_t e = 0; e < n_expert; e++) probs[e] = std::exp(l[e] - mx);
        float sum = 0.0f;
        for (size_t e = 0; e < n_expert; e++) sum += probs[e];
        if (sum > 0.0f)
            for (size_t e = 0; e < n_expert; e++) probs[e] /= sum;
        // L57-62: descending order, keep top_k (ties: lower index first).
        for (size_t e = 0; e < n_expert; e++) order[e] = (int32_t)e;
        std::stable_sort(order.begin(), order.end(), [&](int32_t a, int32_t b) { return probs[a] > probs[b]; });
        float s = 0.0f;
        for (size_t j = 0; j < top_k; j++) {
            ids[t * top_k + j] = order[j];
            weights[t * top_k + j] = probs[order[j]];
        }
        // L64-67: renormalize the kept weights.
        if (normalize) {
            for (size_t j = 0; j < top_k; j++) s += weights[t * top_k + j];
            if (s > 0.0f)
                for (size_t j = 0; j < top_k; j++) weights[t * top_k + j] /= s;
        }
    }
    return RCE_QMM_OK;
}

}  // extern "C"

namespace {

// The grouped experts: h = silu(W1 x) (w3 == nullptr, the benchmark's
// two-matrix expert) or h = silu(W1 x) * (W3 x) (SwiGLU: W1 = gate, W3 =
// up), y = W2 h, out = the decision-order combine.
rce_qmm_status moe_run(rce_qmm_context *ctx, const rce_qmm_weight *const *w1, const rce_qmm_weight *const *w3,
                       const rce_qmm_weight *const *w2, size_t n_expert, const float *x_dev, size_t t_rows,
                       const int32_t *ids_dev, const float *weights_dev, size_t top_k, float *out_dev,
                       rce_qmm_mode mode, void *stream) {
    if (!ctx || !w1 || !w2) return fail(RCE_QMM_NULL_ARGUMENT, "null context or weight list");
    if (n_expert == 0 || n_expert > 4096 || top_k == 0 || top_k > n_expert)
        return fail(RCE_QMM_BAD_SHAPE, "need 0 < top_k <= n_expert <= 4096");
    rce_qmm_status st;
    for (size_t e = 0; e < n_expert; e++) {
        if ((st = check_weight_ctx(ctx, w1[e])) || (st = check_weight_ctx(ctx, w2[e]))) return st;
        if (w3 && (st = check_weight_ctx(ctx, w3[e]))) return st;
    }
    const DevWeight &a1 = w1[0]->dw, &a2 = w2[0]->dw;
    const size_t d_model = a1.n_cols, d_ff = a1.n_rows;
    if (a2.n_rows != d_model || a2.n_cols != d_ff) return fail(RCE_QMM_BAD_SHAPE, "w2 must be [d_model, d_ff] of w1's d_ff");
    for (size_t e = 0; e < n_expert; e++) {
        const DevWeight &b1 = w1[e]->dw, &b2 = w2[e]->dw;
        if (b1.dtype != a1.dtype || b1.n_rows != d_ff || b1.n_cols != d_model || b1.layout != a1.layout ||
            b2.dtype != a2.dtype || b2.n_rows != d_model || b2.n_cols != d_ff || b2.layout != a2.layout)
            return fail(RCE_QMM_BAD_SHAPE, "experts differ in dtype or shape");
        if (w3) {
            const DevWeight &b3 = w3[e]->dw;
            if (b3.dtype != a1.dtype || b3.n_rows != d_ff || b3.n_cols != d_model || b3.layout != a1.layout)
                return fail(RCE_QMM_BAD_SHAPE, "up matrices must match the gate matrices in dtype and shape");
        }
    }
    // the grouped GEMM (F16_MFMA): the nibble kernel for Q4_K / Q5_K / Q4_0 /
    // Q4_1 / Q5_0 (any tile) and Q8_0 / Q6_K (128-row tiles) with K a
    // multiple of 256, the generic one for the rest (Q8_0 / Q5_0 / Q4_1 at
    // other K, F16, BF16 and F32)
    auto experts_ok = [&](uint32_t dt, size_t k) { return supports_mode(dt, k, (int)mode); };
    if (!experts_ok(a1.dtype, d_model) || !experts_ok(a2.dtype, d_ff))
        return fail(RCE_QMM_UNSUPPORTED_DTYPE, "the experts' dtype/shape has no GPU kernel in mode " +
                                                   std::to_string((int)mode));
    if (t_rows == 0) return RCE_QMM_OK;
    if (!x_dev || !ids_dev || !weights_dev || !out_dev) return fail(RCE_QMM_NULL_ARGUMENT, "null device buffer");
    // the nibble kernel's offsets are 32-bit: past that the generic kernel,
    // where it takes the format
    const bool fit1 = gemm_shape_ok(t_rows, a1), fit2 = gemm_shape_ok(t_rows * top_k, a2);
    const bool nib1 = fit1 && gemm_supports(a1.dtype, d_model), nib2 = fit2 && gemm_supports(a2.dtype, d_ff);
    const bool q8n1 = fit1 && gemm_q8_supports(a1.dtype, d_model), q8n2 = fit2 && gemm_q8_supports(a2.dtype, d_ff);
    if (mode == RCE_QMM_MODE_F16_MFMA && ((!nib1 && !q8n1 && !gemm_gen_supports(a1.dtype, d_model)) ||
                                          (!nib2 && !q8n2 && !gemm_gen_supports(a2.dtype, d_ff))))
        return fail(RCE_QMM_BAD_SHAPE, "the grouped Q4_K / Q4_0 GEMM takes below 2^32 bytes of f16 activations per "
                                       "call (t_rows * d_model * 2 and t_rows * top_k * d_ff * 2)");
    if ((st = set_device(ctx->device))) return st;
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;

    // 1. stable grouping of the (token, decision) pairs by expert
    const size_t n_pairs = t_rows * top_k;
    if (n_pairs >= (size_t)1 << 30) return fail(RCE_QMM_BAD_SHAPE, "too many (token, decision) pairs");
    // tile rows of the grouped GEMM for the average rows per expert (the
    // generic kernel takes any tile of at most 128 rows; Q8_0 / Q6_K on the
    // nibble kernel only 128)
    const int bm = (nib1 || nib2) && !q8n1 && !q8n2 ? gemm_tile_rows((n_pairs + n_expert - 1) / n_expert, true) : 128;
    const int max_tiles = (int)(n_pairs / bm + n_expert);
    const size_t meta_ints = (n_expert + 1) + 2 * n_pairs + 2;
    const size_t meta_bytes = align_up(meta_ints * 4, 16) + (size_t)max_tiles * sizeof(MoeTile);
    if ((st = ensure(ctx, ctx->moe_meta, meta_bytes, s))) return st;
    int *offs = static_cast<int *>(ctx->moe_meta.p);
    int *slot_of_pair = offs + n_expert + 1;
    int *tok_of_slot = slot_of_pair + n_pairs;
    int *n_tiles = tok_of_slot + n_pairs;
    int *status = n_tiles + 1;
    MoeTile *tiles = reinterpret_cast<MoeTile *>(static_cast<char *>(ctx->moe_meta.p) + align_up(meta_ints * 4, 16));
    const int *n_slots = offs + n_expert;  // device count of slots with a valid expert
    // expert outputs in slot order
    if ((st = ensure(ctx, ctx->moe_y, n_pairs * d_model * sizeof(float), s))) return st;
    float *y = static_cast<float *>(ctx->moe_y.p);

    if (mode == RCE_QMM_MODE_F16_MFMA) {
        // 2. expert tables (uploaded when the expert set changes)
        std::vector<DevWeight> tab((w3 ? 3 : 2) * n_expert);
        for (size_t e = 0; e < n_expert; e++) {
            tab[e] = w1[e]->dw;
            tab[n_expert + e] = w2[e]->dw;
            if (w3) tab[2 * n_expert + e] = w3[e]->dw;
        }
        const size_t tab_bytes = tab.size() * sizeof(DevWeight);
        if (ctx->moe_wtab_host.size() != tab.size() ||
            std::memcmp(ctx->moe_wtab_host.data(), tab.data(), tab_bytes) != 0) {
            if ((st = ensure(ctx, ctx->moe_wtab, tab_bytes, s))) return st;
            HIP_TRY(hipStreamSynchronize(s));  // no kernel still reads the old table
            HIP_TRY(hipMemcpy(ctx->moe_wtab.p, tab.data(), tab_bytes, hipMemcpyHostToDevice));
            ctx->moe_wtab_host = tab;
        }
        const DevWeight *wtab1 = static_cast<const DevWeight *>(ctx->moe_wtab.p), *wtab2 = wtab1 + n_expert;
        const DevWeight *wtab3 = wtab1 + 2 * n_expert;
        // 3. the grouping, and x -> f16 in the same launch; W1 GEMM on the
        // rows gathered per slot, storing f16 silu(W1 x) (SwiGLU: the gate
        // products in f32, then the up GEMM stores f16 silu(g) * u)
        if ((st = ensure(ctx, ctx->moe_x, t_rows * d_model * 2, s))) return st;
        if ((st = ensure(ctx, ctx->moe_h16, n_pairs * d_ff * 2, s))) return st;
        HIP_TRY(launch_moe_group(ids_dev, n_pairs, (int)top_k, (int)n_expert, bm, offs, slot_of_pair, tok_of_slot,
                                 tiles, n_tiles, status, x_dev, ctx->moe_x.p, t_rows * d_model, s));
        auto grouped = [&](bool nibble, const DevWeight &w, const DevWeight *wtab, const void *a, size_t a_rows,
                           const int *gather, int epi, void *out, const float *aux) {
            return nibble
                       ? launch_gemm_f16_grouped(w, wtab, a, a_rows, gather, tiles, n_tiles, max_tiles, bm, epi, out, aux, s)
                       : launch_gemm_gen_grouped(w, wtab, a, a_rows, gather, tiles, n_tiles, max_tiles, epi, out, aux, s);
        };
        if (w3) {
            if ((st = ensure(ctx, ctx->moe_h, n_pairs * d_ff * sizeof(float), s))) return st;
            float *g = static_cast<float *>(ctx->moe_h.p);
            HIP_TRY(grouped(nib1 || q8n1, a1, wtab1, ctx->moe_x.p, t_rows, tok_of_slot, GEPI_F32, g, nullptr));
            HIP_TRY(grouped(nib1 || q8n1, a1, wtab3, ctx->moe_x.p, t_rows, tok_of_slot, GEPI_SWIGLU_F16, ctx->moe_h16.p, g));
        } else {
            HIP_TRY(grouped(nib1 || q8n1, a1, wtab1, ctx->moe_x.p, t_rows, tok_of_slot, GEPI_SILU_F16, ctx->moe_h16.p,
                            nullptr));
        }
        // 4. W2 GEMM on the slots themselves
        HIP_TRY(grouped(nib2 || q8n2, a2, wtab2, ctx->moe_h16.p, n_pairs, nullptr, GEPI_F32, y, nullptr));
    } else {
        if (mode != RCE_QMM_MODE_EXACT && mode != RCE_QMM_MODE_Q8) return fail(RCE_QMM_BAD_SHAPE, "unknown mode");
        HIP_TRY(launch_moe_group(ids_dev, n_pairs, (int)top_k, (int)n_expert, bm, offs, slot_of_pair, tok_of_slot,
                                 tiles, n_tiles, status, nullptr, nullptr, 0, s));
        if ((st = ensure(ctx, ctx->moe_h, n_pairs * d_ff * sizeof(float), s))) return st;
        float *h = static_cast<float *>(ctx->moe_h.p);
        float *u = nullptr;  // SwiGLU: the up products
        if (w3) {
            if ((st = ensure(ctx, ctx->moe_u, n_pairs * d_ff * sizeof(float), s))) return st;
            u = static_cast<float *>(ctx->moe_u.p);
        }
        // The decode kernels take host row counts: read the grouping back.
        std::vector<int> hoffs(n_expert + 1), hstatus(1);
        HIP_TRY(hipMemcpyAsync(hoffs.data(), offs, hoffs.size() * 4, hipMemcpyDeviceToHost, s));
        HIP_TRY(hipMemcpyAsync(hstatus.data(), status, 4, hipMemcpyDeviceToHost, s));
        HIP_TRY(hipStreamSynchronize(s));
        if (hstatus[0]) return fail(RCE_QMM_BAD_SHAPE, "an expert id is out of range");
        // 2. gather x per slot (f32, the reference's activations)
        if ((st = ensure(ctx, ctx->moe_x, n_pairs * d_model * sizeof(float), s))) return st;
        float *xg = static_cast<float *>(ctx->moe_x.p);
        HIP_TRY(launch_gather_rows(x_dev, tok_of_slot, n_slots, n_pairs, d_model, xg, s));
        // 3. per expert: h = silu(W1 x) [* (W3 x)], y = W2 h (the reference's per-row products).
        // Q8 with several tokens quantizes each launch's activations once
        // (launch_gemv_q8_pre; the launches are ordered on the stream, so
        // they share one workspace).
        size_t n_max = 0;
        for (size_t e = 0; e < n_expert; e++) n_max = std::max<size_t>(n_max, (size_t)(hoffs[e + 1] - hoffs[e]));
        const size_t kmax = std::max(d_model, d_ff);
        if (mode == RCE_QMM_MODE_Q8 && n_max >= 2)
            if ((st = ensure(ctx, ctx->act_q, n_max * (kmax + kmax / 8 + kmax / 4), s))) return st;
        auto gemv = [&](const DevWeight &dw, const float *a, size_t n, float *o) {
            if (mode == RCE_QMM_MODE_Q8 && gemv_q8_pre_supports(dw.dtype, dw.n_cols, n))
                return launch_gemv_q8_pre(dw, a, n, o, ctx->act_q.p, s);
            return launch_gemv(dw, a, n, o, (int)mode, s);
        };
        for (size_t e = 0; e < n_expert; e++) {
            const size_t r0 = (size_t)hoffs[e], n = (size_t)(hoffs[e + 1] - hoffs[e]);
            if (n == 0) continue;
            HIP_TRY(gemv(w1[e]->dw, xg + r0 * d_model, n, h + r0 * d_ff));
            if (w3) HIP_TRY(gemv(w3[e]->dw, xg + r0 * d_model, n, u + r0 * d_ff));
        }
        if (w3) HIP_TRY(launch_swiglu_slots(h, u, n_slots, n_pairs, d_ff, s));
        else HIP_TRY(launch_silu_inplace(h, n_slots, n_pairs, d_ff, s));
        for (size_t e = 0; e < n_expert; e++) {
            const size_t r0 = (size_t)hoffs[e], n = (size_t)(hoffs[e + 1] - hoffs[e]);
            if (n == 0) continue;
            HIP_TRY(gemv(w2[e]->dw, h + r0 * d_ff, n, y + r0 * d_model));
        }
    }
    // 5. combine in decision order
    HIP_TRY(launch_moe_combine(y, slot_of_pair, weights_dev, t_rows, (int)top_k, d_model, out_dev, s));
    return RCE_QMM_OK;
}

}  // namespace

extern "C" {

rce_qmm_status rce_qmm_moe_ffn_dev(rce_qmm_context *ctx, const rce_qmm_weight *const *w1,
                                   const rce_qmm_weight *const *w2, size_t n_expert, const float *x_dev,
                                   size_t t_rows, const int32_t *ids_dev, const float *weights_dev, size_t top_k,
                                   float *out_dev, rce_qmm_mode mode, void *stream) {
    return moe_run(ctx, w1, nullptr, w2, n_expert, x_dev, t_rows, ids_dev, weights_dev, top_k, out_dev, mode, stream);
}

rce_qmm_status rce_qmm_moe_swiglu_dev(rce_qmm_context *ctx, const rce_qmm_weight *const *gate,
                                      const rce_qmm_weight *const *up, const rce_qmm_weight *const *down,
                                      size_t n_expert, const float *x_dev, size_t t_rows, const int32_t *ids_dev,
                                      const float *weights_dev, size_t top_k, float *out_dev, rce_qmm_mode mode,
                                      void *stream) {
    if (!up) return fail(RCE_QMM_NULL_ARGUMENT, "null up-projection list");
    return moe_run(ctx, gate, up, down, n_expert, x_dev, t_rows, ids_dev, weights_dev, top_k, out_dev, mode, stream);
}

rce_qmm_status rce_qmm_dev_alloc(rce_qmm_context *ctx, size_t bytes, void **out) {
    if (!ctx || !out) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    rce_qmm_status st = set_device(ctx->device);
    if (st) return st;
    hipError_t e = hipMalloc(out, std::max<size_t>(bytes, 1));
    if (e != hipSuccess) return fail(RCE_QMM_OUT_OF_MEMORY, std::string("hipMalloc: ") + hipGetErrorString(e));
    return RCE_QMM_OK;
}

rce_qmm_status rce_qmm_dev_free(rce_qmm_context *ctx, void *p) {
    if (!ctx) return fail(RCE_QMM_NULL_ARGUMENT, "null context");
    if (!p) return RCE_QMM_OK;
    rce_qmm_status st = set_device(ctx->device);
    if (st) return st;
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    HIP_TRY(hipFree(p));
    return RCE_QMM_OK;
}

rce_qmm_status rce_qmm_memcpy_h2d(rce_qmm_context *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || ((!dst || !src) && bytes)) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    rce_qmm_status st = set_device(ctx->device);
    if (st) return st;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return RCE_QMM_OK;
}

rce_qmm_status rce_qmm_memcpy_d2h(rce_qmm_context *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || ((!dst || !src) && bytes)) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    rce_qmm_status st = set_device(ctx->device);
    if (st) return st;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return RCE_QMM_OK;
}

}  // extern "C"

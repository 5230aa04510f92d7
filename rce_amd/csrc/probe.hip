// probe.hip -- rce_qmm_read_ceiling_dev: one launch that reads a device
// buffer once, as fast as the chip allows, and does nothing else.  It has
// no counterpart in the reference: it measures the HBM read rate a single
// decode-GEMV launch of the same byte count could reach (launch cost,
// ramp-up and drain included), the ceiling the GEMVs are compared with
// besides the 8 TB/s datasheet peak.
//
// Every variant reads the buffer in 16-byte loads, a wave's load covering
// 1 KB of contiguous memory, all of a thread's loads issued before any is
// used; the loaded words are XOR-folded and written only if they match a
// constant no buffer of interest holds (so no load can be dropped).
#include "abi_internal.h"

namespace {

using rce_qmm_abi::fail;
typedef unsigned v4u __attribute__((ext_vector_type(4)));

// One pass: block b reads [b NT L, (b + 1) NT L) 16-byte words, load i of
// thread t at word b NT L + i NT + t; indices past the end read word 0.
template <int NT, int L, bool NTL>
__global__ __launch_bounds__(NT) void k_read_once(const uint4 *__restrict__ p, size_t n16, unsigned *__restrict__ sink) {
    const size_t base = (size_t)blockIdx.x * NT * L + threadIdx.x;
    uint4 v[L];
#pragma unroll
    for (int i = 0; i < L; i++) {
        const size_t j = base + (size_t)i * NT;
        const uint4 *q = p + (j < n16 ? j : 0);
        if constexpr (NTL) {
            const v4u t = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(q));
            v[i] = make_uint4(t.x, t.y, t.z, t.w);
        } else {
            v[i] = *q;
        }
    }
    unsigned acc = 0;
#pragma unroll
    for (int i = 0; i < L; i++) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

// Grid-stride: a fixed number of blocks, each iteration of a thread issues
// L loads at stride NT before folding them.
template <int NT, int L>
__global__ __launch_bounds__(NT) void k_read_loop(const uint4 *__restrict__ p, size_t n16, unsigned *__restrict__ sink) {
    unsigned acc = 0;
    const size_t step = (size_t)gridDim.x * NT * L;
    for (size_t base = (size_t)blockIdx.x * NT * L + threadIdx.x; base < n16; base += step) {
        uint4 v[L];
#pragma unroll
        for (int i = 0; i < L; i++) {
            const size_t j = base + (size_t)i * NT;
            v[i] = p[j < n16 ? j : 0];
        }
#pragma unroll
        for (int i = 0; i < L; i++) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

__global__ void k_empty(unsigned *sink) {
    if (threadIdx.x == 1024) sink[0] = 0;  // never true: an empty launch of one block
}

template <int NT, int L, bool NTL>
hipError_t once(const uint4 *p, size_t n16, unsigned *sink, hipStream_t s) {
    const size_t per = (size_t)NT * L;
    const size_t blocks = (n16 + per - 1) / per;
    if (blocks == 0 || blocks > 0x7fffffffu) return hipErrorInvalidValue;
    hipLaunchKernelGGL((k_read_once<NT, L, NTL>), dim3((unsigned)blocks), dim3(NT), 0, s, p, n16, sink);
    return hipGetLastError();
}

template <int NT, int L>
hipError_t loop(const uint4 *p, size_t n16, unsigned blocks, unsigned *sink, hipStream_t s) {
    hipLaunchKernelGGL((k_read_loop<NT, L>), dim3(blocks), dim3(NT), 0, s, p, n16, sink);
    return hipGetLastError();
}

// Issue-rate probes: each wave times (s_memtime, shader clocks) 16 * `iters`
// repetitions of one instruction pattern; cyc[block] receives the block's
// slowest wave's cycle count.  The patterns (per repetition):
//   0: eight independent v_fma_f32 chains (8 instructions per iteration);
//   1: one dependent v_add_f32 chain (8 per iteration);
//   2: v_mfma_f32_32x32x16_f16 on four independent accumulators (4 per iteration);
//   3: pattern 2 with 32 independent v_pk_fma_f16 between the MFMAs (4 + 32);
//   4: four v_cvt_scalef32_pk_f32_fp8 (8 values) and 8 adds;
//   5: eight v_cvt_f32_ubyte (8 values) and 8 adds.
typedef _Float16 half8p __attribute__((ext_vector_type(8)));
typedef _Float16 half2p __attribute__((ext_vector_type(2)));
typedef float f32x16p __attribute__((ext_vector_type(16)));
typedef float f32x2p __attribute__((ext_vector_type(2)));
template <int KIND>
__global__ __launch_bounds__(1024) void k_issue(unsigned long long *__restrict__ cyc, float *__restrict__ sink, int iters) {
    const float seed = (float)threadIdx.x * 1e-3f;
    float a[8];
#pragma unroll
    for (int j = 0; j < 8; j++) a[j] = seed + (float)j;
    half8p ha = {1, 2, 3, 4, 5, 6, 7, 8}, hb = ha;
    ha[0] = (_Float16)seed;
    f32x16p c0 = {}, c1 = {}, c2 = {}, c3 = {};
    half2p hv[8];
#pragma unroll
    for (int j = 0; j < 8; j++) hv[j] = half2p{(_Float16)seed, (_Float16)j};
    const half2p hm = {(_Float16)1.001f, (_Float16)0.999f}, hc = {(_Float16)0.01f, (_Float16)0.02f};
    unsigned x = threadIdx.x * 2654435761u;
    __syncthreads();
    const unsigned long long t0 = __builtin_amdgcn_s_memtime();
    for (int i = 0; i < iters; i++) {
#pragma unroll
        for (int rep = 0; rep < 16; rep++) {  // 16 repetitions per trip: the loop's own cost is negligible
        if constexpr (KIND == 0) {
#pragma unroll
            for (int j = 0; j < 8; j++) a[j] = __builtin_fmaf(a[j], 1.0000001f, 1e-7f);
        } else if constexpr (KIND == 1) {
#pragma unroll
            for (int j = 0; j < 8; j++) a[0] = a[0] + 1e-7f;
        } else if constexpr (KIND == 2 || KIND == 3) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ha, hb, c0, 0, 0, 0);
            if constexpr (KIND == 3) {
#pragma unroll
                for (int j = 0; j < 16; j++) hv[j & 7] = __builtin_elementwise_fma(hv[j & 7], hm, hc);
            }
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ha, hb, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ha, hb, c2, 0, 0, 0);
            if constexpr (KIND == 3) {
#pragma unroll
                for (int j = 16; j < 32; j++) hv[j & 7] = __builtin_elementwise_fma(hv[j & 7], hm, hc);
            }
            c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ha, hb, c3, 0, 0, 0);
        } else {
            x = x * 1664525u + 1013904223u;
            const unsigned n = x & 0x0F0F0F0Fu, n2 = (x >> 4) & 0x0F0F0F0Fu;
            float v[8];
            if constexpr (KIND == 4) {
                const f32x2p p0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8((int)n, 512.0f, false);
                const f32x2p p1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8((int)n, 512.0f, true);
                const f32x2p p2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8((int)n2, 512.0f, false);
                const f32x2p p3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8((int)n2, 512.0f, true);
                v[0] = p0.x; v[1] = p0.y; v[2] = p1.x; v[3] = p1.y; v[4] = p2.x; v[5] = p2.y; v[6] = p3.x; v[7] = p3.y;
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) { v[j] = (float)((n >> (8 * j)) & 0xFFu); v[4 + j] = (float)((n2 >> (8 * j)) & 0xFFu); }
            }
#pragma unroll
            for (int j = 0; j < 8; j++) a[j] = a[j] + v[j];
        }
        }
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) s += a[j] + (float)hv[j].x;
#pragma unroll
    for (int j = 0; j < 16; j++) s += c0[j] + c1[j] + c2[j] + c3[j];
    if (s == 1234.5f) sink[0] = s;  // keeps the work; practically never true
    // the block's slowest wave (the arbiter favours older waves, so the
    // first wave alone would time itself as if it had the SIMD to itself)
    __shared__ unsigned long long wave_cyc[16];
    if ((threadIdx.x & 63) == 0) wave_cyc[threadIdx.x >> 6] = t1 - t0;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long m = 0;
        for (unsigned w = 0; w < blockDim.x / 64; w++) m = wave_cyc[w] > m ? wave_cyc[w] : m;
        cyc[blockIdx.x] = m;
    }
}

// Cross-block hand-off cost: every block of the launch stores 64 floats;
// MODE 0 ends there; MODE 1 then makes them visible device-wide the
// memory model's way (__threadfence: L2 write-back and invalidate) and
// counts itself in one device-scope counter, and the block that sees the
// count complete reads every block's floats (the last-block-done pattern a
// kernel would use to run a dependent stage without a second launch);
// MODE 2 does the same with agent-scope atomic stores and loads instead of
// the L2 write-back.  The counter is reset by that last block, so every
// launch starts from zero.  No block waits for another (no spin).
template <int MODE>
__global__ __launch_bounds__(256) void k_handoff(float *__restrict__ data, unsigned *__restrict__ cnt,
                                                 float *__restrict__ res, int nblk) {
    const int tid = threadIdx.x;
    __shared__ int last;
    float v = (float)(blockIdx.x * 256 + tid) * 0.001f;
    if (tid < 64) {
        if constexpr (MODE == 2)
            __hip_atomic_store(data + blockIdx.x * 64 + tid, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
            data[blockIdx.x * 64 + tid] = v;
    }
    if constexpr (MODE == 0) return;
    if constexpr (MODE == 1) __threadfence();
    if constexpr (MODE == 2) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
    if (tid == 0) {
        const unsigned old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = old == (unsigned)nblk - 1;
    }
    __syncthreads();
    if (!last) return;
    if constexpr (MODE == 1) __threadfence();
    float sum = 0.0f;
    for (int i = tid; i < nblk * 64; i += 256) {
        float x;
        if constexpr (MODE == 2) x = __hip_atomic_load(data + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else x = data[i];
        sum += x;
    }
    if (tid == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    res[tid] = sum;
}

}  // namespace

/* No counterpart in the reference: cross-block hand-off probe (see k_handoff). */
extern "C" rce_qmm_status rce_qmm_handoff_probe_dev(rce_qmm_context *ctx, int mode, int blocks, void *data_dev,
                                                    void *counter_dev, void *result_dev, void *stream) {
    using namespace rce_qmm_abi;
    if (!ctx || !data_dev || !counter_dev || !result_dev) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    if (blocks <= 0 || blocks > 65536) return fail(RCE_QMM_BAD_SHAPE, "blocks in 1..65536");
    rce_qmm_status st = set_device(ctx->device);
    if (st) return st;
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
    float *d = static_cast<float *>(data_dev), *r = static_cast<float *>(result_dev);
    unsigned *c = static_cast<unsigned *>(counter_dev);
    switch (mode) {
    case 0: hipLaunchKernelGGL(k_handoff<0>, dim3(blocks), dim3(256), 0, s, d, c, r, blocks); break;
    case 1: hipLaunchKernelGGL(k_handoff<1>, dim3(blocks), dim3(256), 0, s, d, c, r, blocks); break;
    case 2: hipLaunchKernelGGL(k_handoff<2>, dim3(blocks), dim3(256), 0, s, d, c, r, blocks); break;
    default: return fail(RCE_QMM_BAD_SHAPE, "hand-off mode must be 0..2");
    }
    HIP_TRY(hipGetLastError());
    return RCE_QMM_OK;
}

/* No counterpart in the reference: instruction issue-rate probes (see k_issue). */
extern "C" rce_qmm_status rce_qmm_issue_rate_dev(rce_qmm_context *ctx, int kind, int threads, int blocks, int iters,
                                                 void *cycles_dev, void *sink_dev, void *stream) {
    using namespace rce_qmm_abi;
    if (!ctx || !cycles_dev || !sink_dev) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    if (blocks <= 0 || blocks > 65536 || iters <= 0 || (threads != 256 && threads != 512 && threads != 1024))
        return fail(RCE_QMM_BAD_SHAPE, "threads 256, 512 or 1024; blocks in 1..65536; iters > 0");
    rce_qmm_status st = set_device(ctx->device);
    if (st) return st;
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
    unsigned long long *c = static_cast<unsigned long long *>(cycles_dev);
    float *sk = static_cast<float *>(sink_dev);
    switch (kind) {
    case 0: hipLaunchKernelGGL(k_issue<0>, dim3(blocks), dim3(threads), 0, s, c, sk, iters); break;
    case 1: hipLaunchKernelGGL(k_issue<1>, dim3(blocks), dim3(threads), 0, s, c, sk, iters); break;
    case 2: hipLaunchKernelGGL(k_issue<2>, dim3(blocks), dim3(threads), 0, s, c, sk, iters); break;
    case 3: hipLaunchKernelGGL(k_issue<3>, dim3(blocks), dim3(threads), 0, s, c, sk, iters); break;
    case 4: hipLaunchKernelGGL(k_issue<4>, dim3(blocks), dim3(threads), 0, s, c, sk, iters); break;
    case 5: hipLaunchKernelGGL(k_issue<5>, dim3(blocks), dim3(threads), 0, s, c, sk, iters); break;
    default: return fail(RCE_QMM_BAD_SHAPE, "issue-rate kind must be 0..5");
    }
    HIP_TRY(hipGetLastError());
    return RCE_QMM_OK;
}

extern "C" rce_qmm_status rce_qmm_read_ceiling_dev(rce_qmm_context *ctx, const void *buf_dev, size_t bytes,
                                                   void *sink_dev, int variant, void *stream) {
    using namespace rce_qmm_abi;
    if (!ctx || !sink_dev || (!buf_dev && bytes)) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    if (bytes % 16 || reinterpret_cast<uintptr_t>(buf_dev) % 16)
        return fail(RCE_QMM_BAD_SHAPE, "the buffer must be 16-byte aligned and a multiple of 16 bytes");
    if (variant != 9 && bytes == 0) return RCE_QMM_OK;
    rce_qmm_status st = set_device(ctx->device);
    if (st) return st;
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
    const uint4 *p = static_cast<const uint4 *>(buf_dev);
    unsigned *sink = static_cast<unsigned *>(sink_dev);
    const size_t n16 = bytes / 16;
    hipError_t e;
    switch (variant) {
    case 0: e = once<256, 4, false>(p, n16, sink, s); break;
    case 1: e = once<256, 8, false>(p, n16, sink, s); break;
    case 2: e = once<256, 16, false>(p, n16, sink, s); break;
    case 3: e = once<1024, 8, false>(p, n16, sink, s); break;
    case 4: e = once<256, 8, true>(p, n16, sink, s); break;
    case 5: e = loop<256, 8>(p, n16, 1024, sink, s); break;
    case 6: e = loop<256, 8>(p, n16, 2048, sink, s); break;
    case 7: e = loop<512, 8>(p, n16, 512, sink, s); break;
    case 8: e = once<512, 4, false>(p, n16, sink, s); break;
    case 9:
        hipLaunchKernelGGL(k_empty, dim3(1), dim3(64), 0, s, sink);
        e = hipGetLastError();
        break;
    default: return fail(RCE_QMM_BAD_SHAPE, "read-ceiling variant must be 0..9");
    }
    HIP_TRY(e);
    return RCE_QMM_OK;
}

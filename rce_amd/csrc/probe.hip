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

}  // namespace

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

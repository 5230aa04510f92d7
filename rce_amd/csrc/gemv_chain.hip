// gemv_chain.hip -- the whole-element formats F32, F16 and BF16.  The
// reference's row sum is one chain over every position of the row
// (rce-op-qmm/src/lib.rs L458-490: acc += a[i] * w[i], i ascending, from
// +0.0), so each lane owns one row and walks it in that order.  Rows sit in
// the 64-row interleave of LAYOUT_IL64_ROWS: chunk c (16 B) of the 64 rows
// of a group is one contiguous 1 KB wave load.  With one wave per 64 rows
// the launch has few waves, so each wave keeps CHAIN_D chunks (16 KB) in
// flight: the loads of stage s + 1 are issued before the chain consumes
// stage s.  Loads past the row's last chunk read chunk 0 (always valid) and
// are not consumed, so no load sits in a branch.
#include "qmm_gemv_kernels.h"

namespace rce_qmm {
namespace {

constexpr int CHAIN_D = 16;  // chunks per stage

template <int DT>
struct ChainFmt {
    static constexpr int E = DT == T_F32 ? 4 : 8;  // values per 16-byte chunk
};

// value e of a chunk: f32 as is, f16 by v_cvt_f32_f16 (exact), bf16 as the
// high half of an f32 (exact)
template <int DT>
__device__ __forceinline__ float chunk_value(const uint4 &v, int e) {
    if constexpr (DT == T_F32) {
        return __uint_as_float(wrd(v, e));
    } else if constexpr (DT == T_F16) {
        const uint32_t x = wrd(v, e >> 1);
        return h2f((e & 1) ? (x >> 16) : (x & 0xFFFFu));
    } else {
        const uint32_t x = wrd(v, e >> 1);
        return __uint_as_float((e & 1) ? (x & 0xFFFF0000u) : (x << 16));
    }
}

template <int DT>
__global__ __launch_bounds__(64) void k_gemv_chain(DevWeight w, const float *__restrict__ A, float *__restrict__ out) {
    constexpr int E = ChainFmt<DT>::E;
    const int lane = threadIdx.x;
    const size_t grp = blockIdx.x, t = blockIdx.y;
    const size_t k = w.n_cols;
    const float *a = A + t * k;
    const uint4 *src = reinterpret_cast<const uint4 *>(w.base + grp * w.group_stride) + lane;
    const int nc = (int)((k + E - 1) / E);  // chunks holding values
    const int nfull = (int)(k / E);
    const int ns = (nc + CHAIN_D - 1) / CHAIN_D;
    float acc = 0.0f;
    uint4 b0[CHAIN_D], b1[CHAIN_D];
    auto load = [&](uint4 *b, int s) {
#pragma unroll
        for (int i = 0; i < CHAIN_D; i++) {
            const int c = s * CHAIN_D + i;
            b[i] = src[(size_t)(c < nc ? c : 0) * 64];
        }
    };
    auto consume = [&](const uint4 *b, int s) {
#pragma unroll
        for (int i = 0; i < CHAIN_D; i++) {
            const int c = s * CHAIN_D + i;
            const float *ac = a + (size_t)c * E;
            if (c < nfull) {
#pragma unroll
                for (int e = 0; e < E; e++) {
                    const float p = ac[e] * chunk_value<DT>(b[i], e);
                    acc = acc + p;
                }
            } else if (c < nc) {  // the row's last, partial chunk
                const int m = (int)(k - (size_t)c * E);
                for (int e = 0; e < m; e++) {
                    const float p = ac[e] * chunk_value<DT>(b[i], e);
                    acc = acc + p;
                }
            }
        }
    };
    load(b0, 0);
    for (int s = 0; s < ns; s += 2) {
        load(b1, s + 1);
        consume(b0, s);
        load(b0, s + 2);
        consume(b1, s + 1);
    }
    const size_t row = grp * 64 + lane;
    if (row < w.n_rows) out[t * w.n_rows + row] = acc;
}

}  // namespace

hipError_t launch_gemv_chain(const DevWeight &w, const float *a, size_t t_rows, float *out, hipStream_t s) {
    if (t_rows == 0 || w.n_rows == 0) return hipSuccess;
    if (w.layout != LAYOUT_IL64_ROWS || t_rows > 65535) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((w.n_rows + 63) / 64), (unsigned)t_rows);
    switch (w.dtype) {
    case T_F32: hipLaunchKernelGGL(k_gemv_chain<T_F32>, grid, dim3(64), 0, s, w, a, out); break;
    case T_F16: hipLaunchKernelGGL(k_gemv_chain<T_F16>, grid, dim3(64), 0, s, w, a, out); break;
    case T_BF16: hipLaunchKernelGGL(k_gemv_chain<T_BF16>, grid, dim3(64), 0, s, w, a, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace rce_qmm

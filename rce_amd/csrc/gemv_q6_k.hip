// gemv_q6_k.hip -- the Q6_K decode kernels (EXACT: one lane per row; Q8).
#include "qmm_gemv_kernels.h"

namespace rce_qmm {
namespace {

// ---------------------------------------------------------------------------
// Q6_K EXACT: one lane per row (the row sum is a single chain).
// ---------------------------------------------------------------------------

// rce-op-qmm/src/lib.rs L425-454, L1667-1705: per half o, l in 0..32, the
// positions l, l+32, l+64, l+96 in order: sumf += ((d sc) q) a.
template <bool LDS>
__device__ __forceinline__ float q6_exact_superblock(const RawQ6_K &b, const float *as, float sumf) {
    const float d = h2f(b.d);
#pragma unroll
    for (int o = 0; o < 2; o++) {
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const float ds1 = d * (float)q6_sc(b.c[12], 8 * o + c), ds2 = d * (float)q6_sc(b.c[12], 8 * o + c + 2);
            const float ds3 = d * (float)q6_sc(b.c[12], 8 * o + c + 4), ds4 = d * (float)q6_sc(b.c[12], 8 * o + c + 6);
            const float n1 = -32.0f * ds1, n2 = -32.0f * ds2, n3 = -32.0f * ds3, n4 = -32.0f * ds4;
#pragma unroll
            for (int lq = 4 * c; lq < 4 * c + 4; lq++) {
                uint32_t u1, u2, u3, u4;
                q6_words(b, o, lq, u1, u2, u3, u4);
                const float *al = as + 128 * o + 4 * lq;
                float x[4][4];  // activations of positions 4 lq + J + 32 m
                if constexpr (LDS) {  // 16-byte broadcast reads
#pragma unroll
                    for (int m = 0; m < 4; m++) {
                        const float4 v = *reinterpret_cast<const float4 *>(al + 32 * m);
                        x[m][0] = v.x; x[m][1] = v.y; x[m][2] = v.z; x[m][3] = v.w;
                    }
                } else {
#pragma unroll
                    for (int m = 0; m < 4; m++)
#pragma unroll
                        for (int j = 0; j < 4; j++) x[m][j] = al[j + 32 * m];
                }
#define Q6_STEP(J)                                                                   \
    sumf = sumf + __builtin_fmaf(ubyte<J>(u1), ds1, n1) * x[0][J];                     \
    sumf = sumf + __builtin_fmaf(ubyte<J>(u2), ds2, n2) * x[1][J];                     \
    sumf = sumf + __builtin_fmaf(ubyte<J>(u3), ds3, n3) * x[2][J];                     \
    sumf = sumf + __builtin_fmaf(ubyte<J>(u4), ds4, n4) * x[3][J];
                Q6_STEP(0) Q6_STEP(1) Q6_STEP(2) Q6_STEP(3)
#undef Q6_STEP
            }
        }
    }
    return sumf;
}

// LDS: the block's four waves share the token's activations staged in LDS
// (k <= Q6_EXACT_LDS_K), read as broadcasts; else they read them from
// global memory.
constexpr size_t Q6_EXACT_LDS_K = 16384;
template <bool LDS>
__global__ __launch_bounds__(256) void k_gemv_exact_q6k(DevWeight w, const float *__restrict__ A,
                                                        float *__restrict__ out) {
    const size_t row = (size_t)blockIdx.x * 256 + threadIdx.x;
    // Lanes past the end recompute the last row (no branch around loads).
    const size_t rr = row < w.n_rows ? row : w.n_rows - 1;
    const int nsb = (int)(w.n_cols / 256);
    const float *a = A + (size_t)blockIdx.y * w.n_cols;
    extern __shared__ float act[];
    if constexpr (LDS) {
        for (size_t i = threadIdx.x; i < w.n_cols; i += 256) act[i] = a[i];
        __syncthreads();
        a = act;
    }
    float sumf = 0.0f;
    RawQ6_K b0, b1;
    ld_q6_k(w, rr, 0, b0);
    int sb = 0;
    for (; sb + 1 < nsb; sb += 2) {
        ld_q6_k(w, rr, sb + 1, b1);
        sumf = q6_exact_superblock<LDS>(b0, a + 256 * sb, sumf);
        if (sb + 2 < nsb) ld_q6_k(w, rr, sb + 2, b0);
        sumf = q6_exact_superblock<LDS>(b1, a + 256 * (sb + 1), sumf);
    }
    if (sb < nsb) sumf = q6_exact_superblock<LDS>(b0, a + 256 * sb, sumf);
    if (row < w.n_rows) out[(size_t)blockIdx.y * w.n_rows + row] = sumf;
}

}  // namespace

hipError_t launch_gemv_q6_k(const DevWeight &w, const GemvGeom &g, const float *a, size_t t_rows, float *out, int mode,
                            hipStream_t s) {
    if (mode == 0) {
        dim3 grid((unsigned)((w.n_rows + 255) / 256), (unsigned)t_rows);
        if (w.n_cols <= Q6_EXACT_LDS_K)
            hipLaunchKernelGGL(k_gemv_exact_q6k<true>, grid, dim3(256), w.n_cols * sizeof(float), s, w, a, out);
        else
            hipLaunchKernelGGL(k_gemv_exact_q6k<false>, grid, dim3(256), 0, s, w, a, out);
        return hipGetLastError();
    }
    return launch_as_tb<Q6_KQ8, true, 2>(w, g, a, t_rows, out, s);
}
hipError_t launch_gemv_fx_q6_k(const FxLaunch &f, const GemvGeom &g, const float *a, int mode, hipStream_t s) {
    if (mode == 0) return hipErrorInvalidValue;  // EXACT Q6_K is one lane per row
    return launch_as_fx_nt<Q6_KQ8<1>, true>(f, g, a, s);
}
}  // namespace rce_qmm

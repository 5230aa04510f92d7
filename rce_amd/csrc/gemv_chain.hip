// gemv_chain.hip -- the whole-element formats F32, F16 and BF16, and I2_S.
// The reference's row sum is one chain over every position of the row
// (rce-op-qmm/src/lib.rs L458-490: acc += a[i] * w[i], i ascending, from
// +0.0; I2_S, L1478-1537: two chains pos / neg over the whole row), so each
// lane owns one row and walks it in that order.  Rows sit in
// the 64-row interleave of LAYOUT_IL64_ROWS: chunk c (16 B) of the 64 rows
// of a group is one contiguous 1 KB wave load.  With one wave per 64 rows
// the launch has few waves, so each wave keeps CHAIN_D chunks (16 KB) in
// flight: the loads of stage s + 1 are issued before the chain consumes
// stage s.  Loads past the row's last chunk read chunk 0 (always valid) and
// are not consumed, so no load sits in a branch.  The token's activations
// are first copied to LDS (k <= CHAIN_MAX_K), where every lane reads the
// same address (a broadcast) instead of holding them in scalar registers.
#include "qmm_gemv_kernels.h"

namespace rce_qmm {
namespace {

constexpr int CHAIN_D = 16;  // chunks per stage
constexpr int I2S_D = 4;     // I2_S: chunks of 64 codes per stage (fully unrolled)

// Copy the token's k activations to LDS (I2_S: position 128 b + 32 s + gp
// to 128 b + 4 gp + s, so the four positions of one code byte are adjacent).
template <bool I2S>
__device__ __forceinline__ void stage_activations(const float *__restrict__ a, size_t k, float *act) {
    for (size_t i = threadIdx.x; i < k; i += 64) {
        size_t d = i;
        if constexpr (I2S) {
            const size_t r = i % 128;
            d = i - r + 4 * (r % 32) + r / 32;
        }
        act[d] = a[i];
    }
    __syncthreads();
}

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
    extern __shared__ float act[];
    stage_activations<false>(A + t * k, k, act);
    const float *a = act;
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
                float av[E];
#pragma unroll
                for (int q = 0; q < E / 4; q++) {  // 16-byte broadcast reads
                    const float4 v = reinterpret_cast<const float4 *>(ac)[q];
                    av[4 * q] = v.x; av[4 * q + 1] = v.y; av[4 * q + 2] = v.z; av[4 * q + 3] = v.w;
                }
#pragma unroll
                for (int e = 0; e < E; e++) {
                    const float p = av[e] * chunk_value<DT>(b[i], e);
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

// I2_S (lib.rs L1478-1537): byte gp of each block of 128 in order, its four
// codes for positions gp, 32 + gp, 64 + gp, 96 + gp (bits 7:6, 5:4, 3:2,
// 1:0); code 2: pos += a, code 0: neg += a.  Chunk c (16 code bytes) is
// bytes 16 (c % 2) .. + 15 of block c / 2.  A chain step adds the
// activation or +0.0, which leaves a chain (never -0.0: it starts at +0.0)
// unchanged.  The row is scale * (pos - neg) with the tensor's scale.
__global__ __launch_bounds__(64) void k_gemv_chain_i2s(DevWeight w, const float *__restrict__ A,
                                                       float *__restrict__ out) {
    const int lane = threadIdx.x;
    const size_t grp = blockIdx.x, t = blockIdx.y;
    const size_t k = w.n_cols;
    extern __shared__ float act[];
    stage_activations<true>(A + t * k, k, act);
    const uint4 *src = reinterpret_cast<const uint4 *>(w.base + grp * w.group_stride) + lane;
    const int nc = (int)(k / 64);
    const int ns = (nc + I2S_D - 1) / I2S_D;
    float pos = 0.0f, neg = 0.0f;
    uint4 b0[I2S_D], b1[I2S_D];
    auto load = [&](uint4 *b, int s) {
#pragma unroll
        for (int i = 0; i < I2S_D; i++) {
            const int c = s * I2S_D + i;
            b[i] = src[(size_t)(c < nc ? c : 0) * 64];
        }
    };
    auto consume = [&](const uint4 *b, int s) {
#pragma unroll
        for (int i = 0; i < I2S_D; i++) {
            const int c = s * I2S_D + i;
            if (c < nc) {
                // LDS holds block c / 2 with the four positions of code byte gp at 4 gp
                const float4 *ab = reinterpret_cast<const float4 *>(act + (size_t)(c >> 1) * 128) + 16 * (c & 1);
#pragma unroll
                for (int g = 0; g < 16; g++) {
                    const uint32_t byte = (wrd(b[i], g >> 2) >> (8 * (g & 3))) & 0xFFu;
                    const float4 a4 = ab[g];
                    const float av4[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
                    for (int slot = 0; slot < 4; slot++) {
                        const uint32_t code = (byte >> (6 - 2 * slot)) & 3u;
                        const uint32_t av = __float_as_uint(av4[slot]);
                        pos = pos + __uint_as_float(code == 2 ? av : 0u);
                        neg = neg + __uint_as_float(code == 0 ? av : 0u);
                    }
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
    const float scale = *reinterpret_cast<const float *>(w.aux);
    const float d = pos - neg;
    if (row < w.n_rows) out[t * w.n_rows + row] = scale * d;
}

}  // namespace

hipError_t launch_gemv_chain(const DevWeight &w, const float *a, size_t t_rows, float *out, hipStream_t s) {
    if (t_rows == 0 || w.n_rows == 0) return hipSuccess;
    if (w.layout != LAYOUT_IL64_ROWS || t_rows > 65535) return hipErrorInvalidValue;
    if (w.n_cols > CHAIN_MAX_K) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((w.n_rows + 63) / 64), (unsigned)t_rows);
    const size_t lds = w.n_cols * sizeof(float);
    switch (w.dtype) {
    case T_F32: hipLaunchKernelGGL(k_gemv_chain<T_F32>, grid, dim3(64), lds, s, w, a, out); break;
    case T_F16: hipLaunchKernelGGL(k_gemv_chain<T_F16>, grid, dim3(64), lds, s, w, a, out); break;
    case T_BF16: hipLaunchKernelGGL(k_gemv_chain<T_BF16>, grid, dim3(64), lds, s, w, a, out); break;
    case T_I2_S: hipLaunchKernelGGL(k_gemv_chain_i2s, grid, dim3(64), lds, s, w, a, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace rce_qmm

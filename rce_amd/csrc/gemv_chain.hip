// gemv_chain.hip -- the whole-element formats F32, F16 and BF16, and I2_S.
// The reference's row sum is one chain over every position of the row
// (rce-op-qmm/src/lib.rs L458-490: acc += a[i] * w[i], i ascending, from
// +0.0; I2_S, L1478-1537: two chains pos / neg over the whole row), so each
// lane owns one row and walks it in that order.  Rows sit in
// the 64-row interleave of LAYOUT_IL64_ROWS: chunk c (16 B) of the 64 rows
// of a group is one contiguous 1 KB wave load.  With one wave per 64 rows
// the launch has few waves and is bound by the bytes each wave keeps in
// flight: a ring of CHAIN_R stages of CHAIN_D chunks, the loads of stage
// s + CHAIN_R - 1 issued before the chain consumes stage s (36 KB per wave
// in flight).  Loads past the row's last chunk read chunk 0 (always valid) and
// are not consumed, so no load sits in a branch.  The token's activations
// are first copied to LDS (k <= CHAIN_MAX_K), where every lane reads the
// same address (a broadcast) instead of holding them in scalar registers.
#include "qmm_gemv_kernels.h"

namespace rce_qmm {
namespace {

constexpr int CHAIN_D = (int)CHAIN_STAGE;  // chunks per stage: rows are padded to whole stages
constexpr int CHAIN_R = 4;   // stages in the ring
constexpr int I2S_D = 4;     // I2_S: chunks of 64 codes per stage (fully unrolled)

// Copy the token's k activations to LDS, zeros up to `kpad` (I2_S:
// position 128 b + 32 s + gp to 128 b + 4 gp + s, so the four positions of
// one code byte are adjacent).
template <bool I2S>
__device__ __forceinline__ void stage_activations(const float *__restrict__ a, size_t k, size_t kpad, float *act) {
    for (size_t i = threadIdx.x; i < kpad; i += 64) {
        size_t d = i;
        if constexpr (I2S) {
            const size_t r = i % 128;
            d = i - r + 4 * (r % 32) + r / 32;
        }
        act[d] = i < k ? a[i] : 0.0f;
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
        typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
        const half2_t h = __builtin_bit_cast(half2_t, wrd(v, e >> 1));
        return (float)((e & 1) ? h.y : h.x);  // v_cvt_f32_f16 of either half: exact
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
    // The row's chunks, padded with zero chunks to whole stages; past k the
    // weights and the staged activations are +0.0, whose product adds +0.0
    // to the chain (exact: the chain starts at +0.0 and is never -0.0).
    const int nc = (int)(w.group_stride / 1024);
    const int ns = nc / CHAIN_D;
    extern __shared__ float act[];
    stage_activations<false>(A + t * k, k, (size_t)nc * E, act);
    const float *a = act;
    const uint4 *src = reinterpret_cast<const uint4 *>(w.base + grp * w.group_stride) + lane;
    float acc = 0.0f;
    uint4 b0[CHAIN_D], b1[CHAIN_D], b2[CHAIN_D], b3[CHAIN_D];
    auto load = [&](uint4 *b, int s) {
#pragma unroll
        for (int i = 0; i < CHAIN_D; i++) {
            const int c = s * CHAIN_D + i;
            b[i] = src[(size_t)(c < nc ? c : 0) * 64];
        }
    };
    auto consume = [&](const uint4 *b, int s) {
        if (s >= ns) return;  // ring loads past the row (clamped to chunk 0): not consumed
#pragma unroll
        for (int i = 0; i < CHAIN_D; i++) {
            const float *ac = a + (size_t)(s * CHAIN_D + i) * E;
            float av[E];
#pragma unroll
            for (int q = 0; q < E / 4; q++) {  // 16-byte broadcast reads
                const float4 v = reinterpret_cast<const float4 *>(ac)[q];
                av[4 * q] = v.x; av[4 * q + 1] = v.y; av[4 * q + 2] = v.z; av[4 * q + 3] = v.w;
            }
#pragma unroll
            for (int e = 0; e < E; e++) {
                float p;
                if constexpr (DT == T_F16) {
                    // fma(w, a, +0.0) on the widened f16 is one v_fma_mix_f32
                    // (no separate convert): the product rounded once, as
                    // v_mul_f32 rounds it.  A zero product is +0.0 here where
                    // the multiply may give -0.0; either adds the same to a
                    // chain that starts at +0.0 and is never -0.0.
                    p = __builtin_fmaf(chunk_value<DT>(b[i], e), av[e], 0.0f);
                } else {
                    p = av[e] * chunk_value<DT>(b[i], e);
                }
                acc = acc + p;
            }
        }
    };
    static_assert(CHAIN_R == 4, "the ring below is unrolled for four stages");
    load(b0, 0);
    load(b1, 1);
    load(b2, 2);
    for (int s = 0; s < ns; s += 4) {
        load(b3, s + 3);
        consume(b0, s);
        load(b0, s + 4);
        consume(b1, s + 1);
        load(b1, s + 5);
        consume(b2, s + 2);
        load(b2, s + 6);
        consume(b3, s + 3);
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
    stage_activations<true>(A + t * k, k, k, act);
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
    // I2_S: k values; the others: the row's padded chunks' values
    const size_t lds = w.dtype == T_I2_S ? w.n_cols * sizeof(float)
                                         : (w.group_stride / 1024) * (w.dtype == T_F32 ? 4 : 8) * sizeof(float);
    if (lds > 65536) return hipErrorInvalidValue;
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

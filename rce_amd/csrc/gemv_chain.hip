// gemv_chain.hip -- the whole-element formats F32, F16 and BF16, and I2_S.
// The reference's row sum is one chain over every position of the row
// (rce-op-qmm/src/lib.rs L458-490: acc += a[i] * w[i], i ascending, from
// +0.0; I2_S, L1478-1537: two chains pos / neg over the whole row), so each
// lane owns one row and walks it in that order.  Rows sit in the 64-row
// interleave of LAYOUT_IL64_ROWS (I2_S: of LAYOUT_I2S_PLANES, below): chunk
// c (16 B) of the 64 rows
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

// Copy the token's k activations to LDS, zeros up to `kpad`.
__device__ __forceinline__ void stage_activations(const float *__restrict__ a, size_t k, size_t kpad, float *act) {
    for (size_t i = threadIdx.x; i < kpad; i += 64) act[i] = i < k ? a[i] : 0.0f;
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
    stage_activations(A + t * k, k, (size_t)nc * E, act);
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
    // The activations of the next two chunks are read ahead (the LDS
    // latency hides behind a chunk's arithmetic), and a chunk's E products
    // are formed before its E dependent adds.
    float anx[2][E];
    auto read_act = [&](int g, float *dst) {
        const float4 *ac = reinterpret_cast<const float4 *>(a + (size_t)(g < ns * CHAIN_D ? g : 0) * E);
#pragma unroll
        for (int q = 0; q < E / 4; q++) {  // 16-byte broadcast reads
            const float4 v = ac[q];
            dst[4 * q] = v.x; dst[4 * q + 1] = v.y; dst[4 * q + 2] = v.z; dst[4 * q + 3] = v.w;
        }
    };
    read_act(0, anx[0]);
    read_act(1, anx[1]);
    auto consume = [&](const uint4 *b, int s) {
        if (s >= ns) return;  // ring loads past the row (clamped to chunk 0): not consumed
#pragma unroll
        for (int i = 0; i < CHAIN_D; i++) {
            float av[E];
#pragma unroll
            for (int e = 0; e < E; e++) {
                av[e] = anx[0][e];
                anx[0][e] = anx[1][e];
            }
            read_act(s * CHAIN_D + i + 2, anx[1]);
            float p[E];
#pragma unroll
            for (int e = 0; e < E; e++) {
                if constexpr (DT == T_F16) {
                    // fma(w, a, +0.0) on the widened f16 is one v_fma_mix_f32
                    // (no separate convert): the product rounded once, as
                    // v_mul_f32 rounds it.  A zero product is +0.0 here where
                    // the multiply may give -0.0; either adds the same to a
                    // chain that starts at +0.0 and is never -0.0.
                    p[e] = __builtin_fmaf(chunk_value<DT>(b[i], e), av[e], 0.0f);
                } else {
                    p[e] = av[e] * chunk_value<DT>(b[i], e);
                }
            }
#pragma unroll
            for (int e = 0; e < E; e++) acc = acc + p[e];
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
// 1:0); code 2: pos += a, code 0: neg += a; the row is scale * (pos - neg)
// with the tensor's scale.  The two chains are independent, so a block has
// two waves over the same 64 rows: wave 0 the pos chain from the P bit
// plane, wave 1 the neg chain from the N plane (LAYOUT_I2S_PLANES), each
// step one bit as a mask on the activation's bits: a or +0.0, and adding
// +0.0 leaves a chain (never -0.0: it starts at +0.0) unchanged.  The
// activations are staged in LDS in the chain order (position 128 b + 32 s +
// gp at 128 b + 4 gp + s) and read as broadcasts; each wave keeps I2S_R
// chunks of its plane in flight.
constexpr int I2S_R = 8;  // chunks (64 elements, 8 bytes per lane) loaded ahead
__global__ __launch_bounds__(128) void k_gemv_chain_i2s(DevWeight w, const float *__restrict__ A,
                                                        float *__restrict__ out) {
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const size_t grp = blockIdx.x, t = blockIdx.y;
    const size_t k = w.n_cols;
    extern __shared__ float act[];  // k activations in chain order (at the end: the neg chains)
    for (size_t i = tid; i < k; i += 128) {
        const size_t r = i % 128;
        act[i - r + 4 * (r % 32) + r / 32] = A[t * k + i];
    }
    __syncthreads();
    const int nc = (int)(k / 64);
    // this wave's plane: 8 bytes per lane per chunk, chunks 1 KB apart
    const uint2 *src = reinterpret_cast<const uint2 *>(w.base + grp * w.group_stride + 512 * (size_t)wv) + lane;
    uint2 ring[I2S_R];
#pragma unroll
    for (int i = 0; i < I2S_R; i++) ring[i] = src[(size_t)(i < nc ? i : 0) * 128];
    float acc = 0.0f;
    // A chunk's 64 activations, read while the previous chunk is summed.
    float4 an[16];
    auto read_act = [&](int c) {
        const float4 *ac = reinterpret_cast<const float4 *>(act + 64 * (size_t)(c < nc ? c : 0));
#pragma unroll
        for (int q = 0; q < 16; q++) an[q] = ac[q];
    };
    read_act(0);
    // Whole rounds of I2S_R chunks and no branch in a round (a load before a
    // branch is waited for at the join): chunks past the end take zero bits
    // (every step adds +0.0).
    for (int c0 = 0; c0 < nc; c0 += I2S_R) {
#pragma unroll
        for (int i = 0; i < I2S_R; i++) {
            const int c = c0 + i;
            const bool live = c < nc;
            uint2 bits = ring[i];
            bits.x = live ? bits.x : 0u;
            bits.y = live ? bits.y : 0u;
            const int cn = c + I2S_R;  // the ring slot's next chunk (past the end: chunk 0, not consumed)
            ring[i] = src[(size_t)(cn < nc ? cn : 0) * 128];
            float4 a[16];
#pragma unroll
            for (int q = 0; q < 16; q++) a[q] = an[q];
            read_act(c + 1);
            // The masked activations first (independent of each other and
            // of the chain), then the chain's 64 dependent adds.
            uint32_t mv[64];
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const float av[4] = {a[q].x, a[q].y, a[q].z, a[q].w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int j = 4 * q + e;
                    // bit j as an all-ones / zero mask: one v_bfe_i32 (kept
                    // as such; the compiler's compare-and-select form takes
                    // three instructions and a hazard wait)
                    uint32_t m;
                    asm("v_bfe_i32 %0, %1, %2, 1" : "=v"(m) : "v"(j < 32 ? bits.x : bits.y), "n"(j & 31));
                    mv[j] = __float_as_uint(av[e]) & m;
                }
            }
#pragma unroll
            for (int j = 0; j < 64; j++) acc = acc + __uint_as_float(mv[j]);
        }
    }
    __syncthreads();  // both chains done with the activations
    if (wv == 1) act[lane] = acc;
    __syncthreads();
    if (wv != 0) return;
    const size_t row = grp * 64 + lane;
    const float scale = *reinterpret_cast<const float *>(w.aux);
    const float d = acc - act[lane];
    if (row < w.n_rows) out[t * w.n_rows + row] = scale * d;
}

}  // namespace

hipError_t launch_gemv_chain(const DevWeight &w, const float *a, size_t t_rows, float *out, hipStream_t s) {
    if (t_rows == 0 || w.n_rows == 0) return hipSuccess;
    const bool i2s = w.dtype == T_I2_S;
    if (w.layout != (i2s ? LAYOUT_I2S_PLANES : LAYOUT_IL64_ROWS) || t_rows > 65535) return hipErrorInvalidValue;
    if (w.n_cols > CHAIN_MAX_K || (i2s && w.n_cols % 128)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((w.n_rows + 63) / 64), (unsigned)t_rows);
    // I2_S: k values; the others: the row's padded chunks' values
    const size_t lds = i2s ? w.n_cols * sizeof(float) : (w.group_stride / 1024) * (w.dtype == T_F32 ? 4 : 8) * sizeof(float);
    if (lds > 65536) return hipErrorInvalidValue;
    switch (w.dtype) {
    case T_F32: hipLaunchKernelGGL(k_gemv_chain<T_F32>, grid, dim3(64), lds, s, w, a, out); break;
    case T_F16: hipLaunchKernelGGL(k_gemv_chain<T_F16>, grid, dim3(64), lds, s, w, a, out); break;
    case T_BF16: hipLaunchKernelGGL(k_gemv_chain<T_BF16>, grid, dim3(64), lds, s, w, a, out); break;
    case T_I2_S: hipLaunchKernelGGL(k_gemv_chain_i2s, grid, dim3(128), lds, s, w, a, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace rce_qmm

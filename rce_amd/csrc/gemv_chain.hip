// gemv_chain.hip -- the whole-element formats F32, F16 and BF16, and I2_S.
// The reference's row sum is one chain over every position of the row
// (rce-op-qmm/src/lib.rs L458-490: acc += a[i] * w[i], i ascending, from
// +0.0; I2_S, L1478-1537: two chains pos / neg over the whole row), so one
// lane owns each chain and adds in that order.  Rows sit in the 64-row
// interleave of LAYOUT_IL64_ROWS (I2_S: of LAYOUT_I2S_PLANES, below): chunk
// c (16 B) of the 64 rows of a group is one contiguous 1 KB read.  The
// token's activations are first copied to LDS (k <= CHAIN_MAX_K), where
// every lane reads the same address (a broadcast).
#include "gemv_chain_pipe.h"
#include "lds_limit.h"
#include "qmm_gemv_kernels.h"

namespace rce_qmm {
namespace {

constexpr int CHAIN_D = (int)CHAIN_STAGE;  // chunks per stage: rows are padded to whole stages
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
        // volatile: left to itself the scheduler widens every chunk of the
        // helpers' load ring at the top of the loop and runs out of registers
        const uint32_t x = wrd(v, e >> 1);
        uint32_t r;
        if (e & 1)
            asm volatile("v_and_b32 %0, 0xffff0000, %1" : "=v"(r) : "v"(x));
        else
            asm volatile("v_lshlrev_b32 %0, 16, %1" : "=v"(r) : "v"(x));
        return __uint_as_float(r);
    }
}

// One block serves RB rows (16, 32 or 64) of a 64-row group.  Wave 0 holds
// the chains (lane r < RB: row r; the other lanes repeat lane r % RB's
// reads and store nothing); waves 1..H (chain_helpers) form the products.  A
// stage is CHAIN_D chunks (the row padding unit), SV = CHAIN_D * E values.
// The helpers write stage s's products to LDS slot s % 2 and meet the chain
// at barrier s; after it the chain issues the reads of stage s and adds
// stage s - 1's, which it read after the previous barrier (so the helpers
// may overwrite that slot with stage s + 1's products meanwhile).  The
// chain wave so issues only its adds and one 16-byte LDS read per four of
// them; everything else (weight loads, widening, products) runs beside it.
// Each helper keeps CHAIN_DS stages of its weight loads in flight, the
// first ones issued before the activations are staged.
constexpr int CHAIN_SLOTS = 2;
// Helper waves per block: one per row group of 16, but three for 64 rows
// (four waves in all, one per SIMD: a fifth would share the chain's SIMD,
// and the chain, which every barrier waits for, would get half its issue
// slots); stages of loads each helper keeps in flight.
constexpr int chain_helpers(int rb) { return rb == 64 ? 3 : rb / 16; }
constexpr int chain_depth(int rb) { return rb == 64 ? 6 : 8; }

template <int DT, int RB>
__global__ __launch_bounds__(64 * (1 + chain_helpers(RB))) void k_gemv_chain(DevWeight w, const float *__restrict__ A,
                                                                             float *__restrict__ out) {
    constexpr int E = ChainFmt<DT>::E;
    constexpr int G = CHAIN_D;       // chunks per stage
    constexpr int SV = G * E;        // values per stage
    constexpr int H = chain_helpers(RB);
    constexpr int CHAIN_DS = chain_depth(RB);
    constexpr int NT = 64 * (1 + H);
    constexpr int CPL = 64 / RB;     // chunks per wave-wide load
    constexpr int WLH = G / (CPL * H);  // wave-wide loads per helper per stage
    static_assert(WLH * CPL * H == G, "a stage is whole wave-wide loads of every helper");
    constexpr int R = CHAIN_DS * WLH;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const size_t t = blockIdx.y, row0 = (size_t)blockIdx.x * RB;
    const size_t k = w.n_cols;
    // The row's chunks, padded with zero chunks to whole stages; past k the
    // weights and the staged activations are +0.0, whose product adds +0.0
    // to the chain (exact: the chain starts at +0.0 and is never -0.0).
    const int nc = (int)(w.group_stride / 1024);
    const int ns = nc / G;
    const int s_tot = (ns + CHAIN_DS - 1) / CHAIN_DS * CHAIN_DS;  // stages run (whole ring rounds)
    extern __shared__ float lds[];
    float *act = lds;  // nc * E values, then a 16-byte dump slot for the staging's overshoot
    float4 *prod = reinterpret_cast<float4 *>(lds + (size_t)nc * E + 4);  // [CHAIN_SLOTS][SV / 4][RB]
    const int r = lane % RB;
    // helpers: wave-wide load j of helper hw is stage j / WLH, and within it
    // chunks (i H + hw) CPL .. + CPL - 1 for i = j % WLH (this lane's: + lane / RB)
    const int hw = wv - 1, cl = lane / RB;
    // Buffer loads from the group's base: the lane's part of the offset in
    // one VGPR, the wave-wide load's part in an SGPR.  Stages past the row
    // load the last stage again (not used); a clamp, not a test: a load
    // under a branch is waited for where the branch joins.
    const WBuf wb = make_wbuf(w.base + (row0 / 64) * w.group_stride, (uint32_t)((row0 % 64 + r) * 16 + cl * 1024));
    auto soff_of = [&](int j) -> uint32_t {
        const int s = j / WLH, i = j - s * WLH;
        return (uint32_t)(min(s, ns - 1) * G + (i * H + hw) * CPL) * 1024u;
    };
    uint4 ring[R];
    if (wv != 0) {
#pragma unroll
        for (int j = 0; j < R; j++) ring[j] = bld16(wb, 0, soff_of(j));
    }
    // the token's activations, zeros up to the padded row
    stage_act<NT, 24>(A + t * k, k, (size_t)nc * E, act, [](size_t i) { return i; });
    __syncthreads();
    if (wv == 0) {
        const float acc = run_chain<SV, RB>(prod + r, ns, s_tot);
        const size_t row = row0 + lane;
        if (lane < RB && row < w.n_rows) out[t * w.n_rows + row] = acc;
        return;
    }
    // helpers: s_tot stages, each ending at a barrier once its products are
    // written.  A stage's activations are read during the stage before (LDS
    // reads issued ahead of that stage's product stores, which the compiler
    // would otherwise wait for: both live in the one LDS array).
    float4 an[2][WLH][E / 4];
    auto read_act = [&](int s, float4 (*dst)[E / 4]) {
        const int sa = min(s, ns - 1);  // stages past the row: the last stage's activations (not used)
#pragma unroll
        for (int i = 0; i < WLH; i++) {
            const int cs = (i * H + hw) * CPL + cl;
            const float4 *ac = reinterpret_cast<const float4 *>(act + (size_t)sa * SV + (size_t)cs * E);
#pragma unroll
            for (int q = 0; q < E / 4; q++) dst[i][q] = ac[q];
        }
    };
    read_act(0, an[0]);
    for (int s0 = 0; s0 < s_tot; s0 += CHAIN_DS) {
#pragma unroll
        for (int u = 0; u < CHAIN_DS; u++) {
            const int s = s0 + u;
            read_act(s + 1, an[(u + 1) & 1]);
            float4 *p = prod + (size_t)(s % CHAIN_SLOTS) * (SV / 4) * RB + r;
#pragma unroll
            for (int i = 0; i < WLH; i++) {
                const uint4 v = ring[u * WLH + i];
                const int cs = (i * H + hw) * CPL + cl;  // chunk within the stage
                float a[E];
#pragma unroll
                for (int q = 0; q < E / 4; q++) {
                    const float4 x = an[u & 1][i][q];
                    a[4 * q] = x.x; a[4 * q + 1] = x.y; a[4 * q + 2] = x.z; a[4 * q + 3] = x.w;
                }
                float pr[E];
#pragma unroll
                for (int e = 0; e < E; e++) {
                    if constexpr (DT == T_F16) {
                        // fma(w, a, +0.0) on the widened f16 is one v_fma_mix_f32
                        // (no separate convert): the product rounded once, as
                        // v_mul_f32 rounds it.  A zero product is +0.0 here where
                        // the multiply may give -0.0; either adds the same to a
                        // chain that starts at +0.0 and is never -0.0.
                        pr[e] = __builtin_fmaf(chunk_value<DT>(v, e), a[e], 0.0f);
                    } else {
                        pr[e] = a[e] * chunk_value<DT>(v, e);
                    }
                }
                // the slot's next load once its value is used (a load into a
                // register still in use would take another register, and the
                // loop's copy back would wait for every load in flight)
                ring[u * WLH + i] = bld16(wb, 0, soff_of((s + CHAIN_DS) * WLH + i));
#pragma unroll
                for (int q = 0; q < E / 4; q++)
                    p[(size_t)(cs * (E / 4) + q) * RB] = make_float4(pr[4 * q], pr[4 * q + 1], pr[4 * q + 2], pr[4 * q + 3]);
            }
            __syncthreads();
        }
    }
}

// I2_S (lib.rs L1478-1537): byte gp of each block of 128 in order, its four
// codes for positions gp, 32 + gp, 64 + gp, 96 + gp (bits 7:6, 5:4, 3:2,
// 1:0); code 2: pos += a, code 0: neg += a; the row is scale * (pos - neg)
// with the tensor's scale.  The activations are staged in LDS in the chain
// order (position 128 b + 32 s + gp at 128 b + 4 gp + s), so element j of a
// row's bit planes (LAYOUT_I2S_PLANES) is the chain's step j.  A block
// serves 32 rows: wave 0 holds the 64 chains (lane l < 32: row l's pos
// chain, lane 32 + l: its neg chain); helper waves 1..4 turn the plane bits
// into the chains' addends, each bit a mask on the activation's bits (a or
// +0.0; adding +0.0 leaves a chain, which starts at +0.0 and is never -0.0,
// unchanged), through LDS as the F32 / F16 / BF16 chains above do.  A
// stage is two 64-element chunks; helper h takes chunk h / 2's plane word
// h % 2 (32 elements) of all 64 chains.
constexpr int I2S_DS = 8;  // stages of plane words a helper keeps in flight

__global__ __launch_bounds__(320) void k_gemv_chain_i2s(DevWeight w, const float *__restrict__ A,
                                                        float *__restrict__ out) {
    constexpr int SV = 128;  // values per stage
    constexpr int NT = 320;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const size_t t = blockIdx.y, row0 = (size_t)blockIdx.x * 32;
    const size_t k = w.n_cols;
    const int ns = (int)(k / SV);
    const int s_tot = (ns + I2S_DS - 1) / I2S_DS * I2S_DS;
    extern __shared__ float lds[];
    float *act = lds;  // k values in chain order, then a 16-byte dump slot
    float4 *prod = reinterpret_cast<float4 *>(lds + k + 4);  // [2][SV / 4][64]
    // helpers: plane word of chain `lane` for stage s: chunk 2 s + h / 2, word h % 2
    const int hw = wv - 1;
    const WBuf wb = make_wbuf(w.base + (row0 / 64) * w.group_stride,
                              (uint32_t)((lane / 32) * 512 + (row0 % 64 + lane % 32) * 8 + (hw & 1) * 4));
    auto soff_of = [&](int s) -> uint32_t { return (uint32_t)(2 * min(s, ns - 1) + (hw >> 1)) * 1024u; };
    uint32_t ring[I2S_DS];
    if (wv != 0) {
#pragma unroll
        for (int j = 0; j < I2S_DS; j++) ring[j] = bld4(wb, 0, soff_of(j));
    }
    // the activations in chain order
    stage_act<NT, 16>(A + t * k, k, k, act, [](size_t i) { const size_t r = i % 128; return i - r + 4 * (r % 32) + r / 32; });
    __syncthreads();
    if (wv == 0) {
        const float acc = run_chain<SV, 64>(prod + lane, ns, s_tot);
        const float neg = __shfl_down(acc, 32);
        const size_t row = row0 + lane;
        const float scale = *reinterpret_cast<const float *>(w.aux);
        if (lane < 32 && row < w.n_rows) out[t * w.n_rows + row] = scale * (acc - neg);
        return;
    }
    // helpers: this helper's 32 steps of every chain per stage; the stage's
    // activations read during the stage before
    const int j0 = (hw >> 1) * 64 + (hw & 1) * 32;  // first step within the stage
    float4 an[2][8];
    auto read_act = [&](int s, float4 *dst) {
        const float4 *ac = reinterpret_cast<const float4 *>(act + (size_t)min(s, ns - 1) * SV + j0);
#pragma unroll
        for (int q = 0; q < 8; q++) dst[q] = ac[q];
    };
    read_act(0, an[0]);
    for (int s0 = 0; s0 < s_tot; s0 += I2S_DS) {
#pragma unroll
        for (int u = 0; u < I2S_DS; u++) {
            const int s = s0 + u;
            read_act(s + 1, an[(u + 1) & 1]);
            const uint32_t bits = ring[u];
            uint32_t mv[32];
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const float4 x = an[u & 1][q];
                const float av[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    // bit 4q + e as an all-ones / zero mask: one v_bfe_i32 (kept
                    // as such; the compiler's compare-and-select form takes
                    // three instructions and a hazard wait).  Volatile, so that
                    // the scheduler keeps each stage's masks in its stage.
                    uint32_t m;
                    asm volatile("v_bfe_i32 %0, %1, %2, 1" : "=v"(m) : "v"(bits), "n"(4 * q + e));
                    mv[4 * q + e] = __float_as_uint(av[e]) & m;
                }
            }
            ring[u] = bld4(wb, 0, soff_of(s + I2S_DS));  // the slot's next word once this one is used
            float4 *p = prod + (size_t)(s & 1) * (SV / 4) * 64 + (size_t)(j0 / 4) * 64 + lane;
#pragma unroll
            for (int q = 0; q < 8; q++)
                p[q * 64] = make_float4(__uint_as_float(mv[4 * q]), __uint_as_float(mv[4 * q + 1]),
                                        __uint_as_float(mv[4 * q + 2]), __uint_as_float(mv[4 * q + 3]));
            __syncthreads();
        }
    }
}

template <int DT, int RB>
hipError_t launch_chain(const DevWeight &w, const float *a, size_t t_rows, float *out, hipStream_t s) {
    constexpr int E = ChainFmt<DT>::E;
    const size_t lds = ((w.group_stride / 1024) * E + 4) * sizeof(float) + (size_t)CHAIN_SLOTS * CHAIN_D * E * RB * sizeof(float);
    if (lds > 64 * 1024) {  // activations of a long row: more than the default 64 KB
        const hipError_t e = ensure_lds_limit((const void *)k_gemv_chain<DT, RB>, 160 * 1024);
        if (e != hipSuccess) return e;
    }
    const dim3 grid((unsigned)((w.n_rows + RB - 1) / RB), (unsigned)t_rows);
    hipLaunchKernelGGL((k_gemv_chain<DT, RB>), grid, dim3(64 * (1 + chain_helpers(RB))), lds, s, w, a, out);
    return hipGetLastError();
}

template <int DT>
hipError_t launch_chain_rb(const DevWeight &w, const float *a, size_t t_rows, float *out, hipStream_t s) {
    // Rows per block: 64 while that leaves a block per CU, else 32 or 16
    // (a chain's time does not depend on how many rows share its wave).
    const size_t groups = (w.n_rows + 63) / 64 * t_rows;
    if (groups >= 256) return launch_chain<DT, 64>(w, a, t_rows, out, s);
    if (2 * groups >= 256) return launch_chain<DT, 32>(w, a, t_rows, out, s);
    return launch_chain<DT, 16>(w, a, t_rows, out, s);
}

}  // namespace

hipError_t chain_prepare_lds() {
    const void *fns[] = {(const void *)k_gemv_chain<T_F32, 16>,  (const void *)k_gemv_chain<T_F32, 32>,
                         (const void *)k_gemv_chain<T_F32, 64>,  (const void *)k_gemv_chain<T_F16, 16>,
                         (const void *)k_gemv_chain<T_F16, 32>,  (const void *)k_gemv_chain<T_F16, 64>,
                         (const void *)k_gemv_chain<T_BF16, 16>, (const void *)k_gemv_chain<T_BF16, 32>,
                         (const void *)k_gemv_chain<T_BF16, 64>, (const void *)k_gemv_chain_i2s};
    for (const void *f : fns) {
        const hipError_t e = ensure_lds_limit(f, 160 * 1024);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_gemv_chain(const DevWeight &w, const float *a, size_t t_rows, float *out, hipStream_t s) {
    if (t_rows == 0 || w.n_rows == 0) return hipSuccess;
    const bool i2s = w.dtype == T_I2_S;
    if (w.layout != (i2s ? LAYOUT_I2S_PLANES : LAYOUT_IL64_ROWS) || t_rows > 65535) return hipErrorInvalidValue;
    if (w.n_cols == 0 || w.n_cols > CHAIN_MAX_K || (i2s && w.n_cols % 128)) return hipErrorInvalidValue;
    if (!i2s && (w.group_stride % (1024 * CHAIN_D) || w.group_stride / 1024 * (w.dtype == T_F32 ? 4 : 8) < w.n_cols))
        return hipErrorInvalidValue;
    switch (w.dtype) {
    case T_F32: return launch_chain_rb<T_F32>(w, a, t_rows, out, s);
    case T_F16: return launch_chain_rb<T_F16>(w, a, t_rows, out, s);
    case T_BF16: return launch_chain_rb<T_BF16>(w, a, t_rows, out, s);
    case T_I2_S: {
        // k activations, the dump slot, two stages of 128 addends of 64 chains
        const size_t lds = (w.n_cols + 4) * sizeof(float) + 2 * 128 * 64 * sizeof(float);
        const hipError_t e = ensure_lds_limit((const void *)k_gemv_chain_i2s, 160 * 1024);
        if (e != hipSuccess) return e;
        const dim3 grid((unsigned)((w.n_rows + 31) / 32), (unsigned)t_rows);
        hipLaunchKernelGGL(k_gemv_chain_i2s, grid, dim3(320), lds, s, w, a, out);
        return hipGetLastError();
    }
    default: return hipErrorInvalidValue;
    }
}

}  // namespace rce_qmm

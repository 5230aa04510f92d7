// gemv_q8_mfma.hip -- the Q8-activation GEMV of several tokens (mode Q8,
// 2..16 tokens per token tile) for Q4_0 and Q8_0 weights on the int8
// matrix cores: each block of 32's exact int32 dot of the weight's integers
// with the token's Q8 activation integers is one lane's element of a
// v_mfma_i32_16x16x32_i8 (16 weight rows x 16 tokens, K = one block), and
// the rest of the Q8 path is the same f32 arithmetic as the decode kernels'
// (qmm_gemv_kernels.h, Q32Q8): Q4_0 sub = dx * (float)(isum - 8 xs), Q8_0
// sub = dx * (float)isum, addend = d * sub, the row sum folded over blocks
// in order from +0.0 (rce-op-qmm/src/lib.rs L496-522 / L648-670 with the
// block sub-sums in Q8 form).  So the result is bit-identical to the
// decode kernels' Q8 mode and to the oracle's orc_mm_batched_q8.
//
// Why: with several tokens the decode kernels hold every token's
// activations in registers, so a block takes at most 4 tokens and the
// weight is streamed once per token group, and every (row, token, block)
// addend goes through LDS to a fold thread.  Here one wave owns 16 rows x
// 16 tokens: the weight is read once for all tokens and the fold stays in
// registers.
//
// Work mapping: one wave per block of 64 threads, owning output rows r0 ..
// r0 + 15 and tokens t0 .. t0 + 15 over all of K.  Lane l: A operand row
// l % 16, k-slice g = l / 16 (positions 8 g .. 8 g + 7 of the block);
// B operand token l % 16, the same k-slice; the accumulator element i is
// row 4 g + i, token l % 16.  Q4_0 positions 8 g .. 8 g + 7 are the low
// (g < 2) or high (g >= 2) nibbles of bytes 8 (g & 1) .. + 7 of the block's
// 16 bytes; Q8_0's are bytes 8 (g & 1) .. of plane 1 (g < 2) or plane 2.
//
// Weights reach LDS by direct-to-LDS buffer loads (no registers), RING
// stages of 8 blocks ahead: a stage is 16 rows x 8 blocks x 16 bytes per
// plane; every fourth stage also loads the 16 rows' scales of four stages.
// The buffer starts at row r0 and ends at row n, so rows past the end read
// zeros.  Activations (the pre-quantized Q8 workspace, L2-resident) are
// loaded into registers one stage ahead.  The explicit vmcnt waits count
// both kinds of load (they retire in order), and the LDS reads are inline
// asm, so the compiler's own waits never cover the whole ring.
#include "qmm_gemv_kernels.h"

namespace rce_qmm {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int SB = 8;     // blocks of 32 per stage
constexpr int RING = 8;   // stages in the LDS ring
constexpr int SGRP = 4;   // stages per scale load (one 16-byte chunk = 8 scales per row and stage)
// scale loads in the ring: the stages in flight span up to 3 groups; a
// group's slot is rewritten 4 groups later, after its last reader
constexpr int SRING = 4;

template <bool Q4>
struct MfmaQ8 {
    static constexpr int NPL = Q4 ? 1 : 2;                 // weight planes
    static constexpr int STAGE_W = NPL * 16 * SB * 16;     // weight bytes of a stage (2 or 4 KB)
    static constexpr int SCALE_GRP = 16 * SGRP * 16;       // one scale load: 1 KB
    static constexpr int LDS = RING * STAGE_W + SRING * SCALE_GRP;
    static constexpr int W_LOADS = NPL * 2;                // DMA instructions of a stage's weights
    // activation loads of a stage: 8 xq (b64), 2 dx (b128), 4 s16 (b128)
    static constexpr int ACT_LOADS = Q4 ? SB + 2 + 4 : SB + 2;
};

__device__ __forceinline__ void buf_load_lds16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                               unsigned char *lds_wave) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds_wave, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t byte_buffer(const void *base, uint32_t n) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)n, 0x00020000);
}
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
template <int OFF>
__device__ __forceinline__ u32x2 lds_read8(uint32_t a) {
    u32x2 v;
    asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v) : "v"(a), "n"(OFF) : "memory");
    return v;
}
template <int OFF>
__device__ __forceinline__ u32x4 lds_read16(uint32_t a) {
    u32x4 v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(a), "n"(OFF) : "memory");
    return v;
}
template <class T>
__device__ __forceinline__ void pin(T &r) {
    asm volatile("" : "+v"(r));
}
// s_waitcnt vmcnt(N) alone (gfx9 encoding: expcnt and lgkmcnt not waited for)
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
// One stage's activations for this lane's token: xq of positions 8 g .. of
// the stage's 8 blocks, dx of the 8 blocks, the 16 half-block sums s16.
struct Act {
    u32x2 xq[SB];
    u32x4 dx[2];
    u32x4 s16[4];
};

template <bool Q4>
__global__ __launch_bounds__(64) void k_gemv_q8_mfma(DevWeight w, const unsigned char *__restrict__ preq, int T,
                                                     float *__restrict__ out) {
    using C = MfmaQ8<Q4>;
    __shared__ __align__(16) unsigned char lds[C::LDS];
    const int lane = threadIdx.x, r16 = lane & 15, g = lane >> 4;
    const size_t n = w.n_rows, k = w.n_cols, nb = k / 32;
    const size_t r0 = (size_t)blockIdx.x * 16;
    const int t0 = blockIdx.y * 16;
    const int nst = (int)(nb / SB);  // stages (the host requires k % 256 == 0)

    // weight buffer from row r0 to the last row: rows past n read zeros
    const size_t nrows = n - r0 < 16 ? n - r0 : 16;
    const __amdgpu_buffer_rsrc_t wb = byte_buffer(w.base + r0 * w.row_stride, (uint32_t)(nrows * w.row_stride));
    // DMA lane offsets: weights instruction j covers blocks 4 j .. 4 j + 3
    // of the stage, lane l row l % 16, block 4 j + l / 16; scales: lane l
    // row l % 16, the 16-byte chunk (8 scales) of stage l / 16 of the group
    const uint32_t w_lane = (uint32_t)r16 * (uint32_t)w.row_stride + 16u * (uint32_t)g;
    const uint32_t s_lane = w_lane;
    unsigned char *ring = lds, *sring = lds + RING * C::STAGE_W;

    // Loads of virtual stage s (past the end: the last stage again, into a
    // slot no later stage reads)
    auto issue = [&](int s, auto u_c) {
        constexpr int u = decltype(u_c)::value;  // s % SGRP
        const int sc = s < nst ? s : nst - 1;
        if constexpr (u == 0) {
            const int grp = sc / SGRP;
            buf_load_lds16(wb, s_lane, (uint32_t)(16 * SGRP * grp), sring + ((s / SGRP) % SRING) * C::SCALE_GRP);
        }
        unsigned char *dst = ring + (s % RING) * C::STAGE_W;
#pragma unroll
        for (int p = 0; p < C::NPL; p++) {
            const uint32_t plane = p == 0 ? (uint32_t)w.plane1 : (uint32_t)w.plane2;
#pragma unroll
            for (int j = 0; j < 2; j++)
                buf_load_lds16(wb, w_lane + plane, (uint32_t)(16 * (SB * sc + 4 * j)), dst + (p * 2 + j) * 1024);
        }
    };
    // this lane's token (lanes past T read token T - 1; their sums are not stored)
    const int tt = t0 + r16 < T ? t0 + r16 : T - 1;
    const ActLds L(const_cast<unsigned char *>(preq), k, T);
    const unsigned char *xq_t = reinterpret_cast<const unsigned char *>(L.xq) + (size_t)tt * k + 8 * g;
    const float *dx_t = L.dx + (size_t)tt * nb;
    const int *s16_t = L.s16 + (size_t)tt * (2 * nb);
    auto act_load = [&](Act &a, int s) {
        const int sc = s < nst ? s : nst - 1;
        const size_t b0 = (size_t)SB * sc;
#pragma unroll
        for (int j = 0; j < SB; j++) a.xq[j] = *reinterpret_cast<const u32x2 *>(xq_t + 32 * (b0 + j));
        a.dx[0] = *reinterpret_cast<const u32x4 *>(dx_t + b0);
        a.dx[1] = *reinterpret_cast<const u32x4 *>(dx_t + b0 + 4);
        if constexpr (Q4) {
#pragma unroll
            for (int j = 0; j < 4; j++) a.s16[j] = *reinterpret_cast<const u32x4 *>(s16_t + 2 * b0 + 4 * j);
        }
    };

    // LDS read addresses: the A operand of block j of a stage at
    // (p * 2 + j / 4) * 1024 + ((j % 4) * 16 + r16) * 16 + 8 (g & 1),
    // plane p = g / 2 for Q8_0; the scales of row 4 g + i at
    // (stage % SGRP * 16 + 4 g + i) * 16.
    const uint32_t ring0 = lds_addr(ring), sring0 = lds_addr(sring);
    const uint32_t a_rd = ring0 + (uint32_t)((Q4 ? 0 : (g >> 1) * 2048) + r16 * 16 + 8 * (g & 1));
    const uint32_t s_rd = sring0 + (uint32_t)(4 * g * 16);
    const int nsh = Q4 ? 4 * (g >> 1) : 0;

    float sumf[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    Act a0, a1;

    // prologue: weights of stages 0 .. RING - 2, activations of stage 0
    issue(0, std::integral_constant<int, 0>{});
    issue(1, std::integral_constant<int, 1>{});
    issue(2, std::integral_constant<int, 2>{});
    issue(3, std::integral_constant<int, 3>{});
    issue(4, std::integral_constant<int, 0>{});
    issue(5, std::integral_constant<int, 1>{});
    issue(6, std::integral_constant<int, 2>{});
    static_assert(RING == 8 && SGRP == 4, "the prologue issues stages 0 .. 6");
    act_load(a0, 0);

    auto stage = [&](int s, auto u_c, const Act &cur, Act &nxt) {
        constexpr int u = decltype(u_c)::value;  // s % SGRP
        constexpr int un = (u + RING - 1) % SGRP;  // (s + RING - 1) % SGRP
        issue(s + RING - 1, std::integral_constant<int, un>{});
        act_load(nxt, s + 1);
        // everything up to this stage's activations (issued one stage ago,
        // after its weights) has arrived: the loads after them are this
        // iteration's weights and activations
        constexpr int after = (C::W_LOADS + (un == 0 ? 1 : 0)) + C::ACT_LOADS;
        wait_vm<after>();
        const uint32_t wst = a_rd + (uint32_t)((s % RING) * C::STAGE_W);
        const uint32_t sst = s_rd + (uint32_t)(((s / SGRP) % SRING) * C::SCALE_GRP + u * 256);
        u32x2 av[SB];
        u32x4 sc[4];
#pragma unroll
        for (int j = 0; j < SB; j++) {
            const uint32_t aa = wst + (uint32_t)((j / 4) * 1024 + (j % 4) * 256);
            av[j] = lds_read8<0>(aa);
        }
        sc[0] = lds_read16<0>(sst);
        sc[1] = lds_read16<16>(sst);
        sc[2] = lds_read16<32>(sst);
        sc[3] = lds_read16<48>(sst);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int j = 0; j < SB; j++) pin(av[j]);
#pragma unroll
        for (int i = 0; i < 4; i++) pin(sc[i]);
#pragma unroll
        for (int j = 0; j < SB; j++) {
            u32x2 aw = av[j];
            if constexpr (Q4) {
                aw.x = (aw.x >> nsh) & 0x0F0F0F0Fu;
                aw.y = (aw.y >> nsh) & 0x0F0F0F0Fu;
            }
            long A, B;
            __builtin_memcpy(&A, &aw, 8);
            __builtin_memcpy(&B, &cur.xq[j], 8);
            const i32x4 acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, i32x4{0, 0, 0, 0}, 0, 0, 0);
            const float dx = __uint_as_float(cur.dx[j / 4][j % 4]);
            int xs8 = 0;
            if constexpr (Q4) xs8 = 8 * ((int)cur.s16[j / 2][2 * (j % 2)] + (int)cur.s16[j / 2][2 * (j % 2) + 1]);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float d = h2f(sc[i][j / 2] >> (16 * (j % 2)));
                const float sub = dx * (float)(acc[i] - xs8);
                const float ad = d * sub;
                sumf[i] = sumf[i] + ad;
            }
        }
    };
    int s = 0;
    for (; s + 4 <= nst; s += 4) {
        stage(s, std::integral_constant<int, 0>{}, a0, a1);
        stage(s + 1, std::integral_constant<int, 1>{}, a1, a0);
        stage(s + 2, std::integral_constant<int, 2>{}, a0, a1);
        stage(s + 3, std::integral_constant<int, 3>{}, a1, a0);
    }
    if (s < nst) stage(s, std::integral_constant<int, 0>{}, a0, a1);
    if (s + 1 < nst) stage(s + 1, std::integral_constant<int, 1>{}, a1, a0);
    if (s + 2 < nst) stage(s + 2, std::integral_constant<int, 2>{}, a0, a1);
    __builtin_amdgcn_s_waitcnt(0);  // no load still writing LDS when the wave ends
    if (t0 + r16 < T) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const size_t row = r0 + 4 * g + i;
            if (row < n) out[(size_t)(t0 + r16) * n + row] = sumf[i];
        }
    }
}

}  // namespace

// The token bound is the decode kernels' pre-quantized form's (this form's
// callers fall back to it), and k_quantize_act counts its tasks,
// t_rows * n_cols / 8, in an int.
bool gemv_q8_mfma_supports(uint32_t dtype, size_t n_cols, size_t t_rows) {
    return (dtype == T_Q4_0 || dtype == T_Q8_0) && n_cols % 256 == 0 && t_rows >= 2 && t_rows <= 65535 * 8 &&
           n_cols * 16 < ((size_t)1 << 31) && t_rows * (n_cols / 8) < ((size_t)1 << 31);
}

// Where this form is the faster one.  A wave walks all of K for its 16 rows
// (the fold is sequential), one wave per 16 rows, so a short K leaves it
// latency-bound at about 1 us per stage of 8 blocks; the decode kernels'
// form re-reads the weight per group of 4 tokens and folds through LDS, which
// costs most at long K and many tokens.  Measured (Q8, us, that form / this
// one): Q4_0 11008x4096 at 2 / 8 / 64 tokens 9.6 / 15.9 / 92.5 against
// 22.6 / 24.6 / 100.8; Q4_0 4096x14336 at 2 / 4 / 8 / 16 / 64 tokens
// 14.9 / 63.6 / 112.8 / 208.0 / 730.1 against 52.7 / 53.9 / 56.2 / 60.5 /
// 109.1; Q8_0 4096x4096 at 64 tokens 37.9 against 35.0.
bool gemv_q8_mfma_preferred(size_t n_cols, size_t t_rows) { return (n_cols >= 8192 && t_rows >= 4) || t_rows >= 64; }

hipError_t launch_gemv_q8_mfma(const DevWeight &w, const unsigned char *preq, size_t t_rows, float *out, hipStream_t s) {
    if (t_rows == 0 || w.n_rows == 0) return hipSuccess;
    if (!gemv_q8_mfma_supports(w.dtype, w.n_cols, t_rows) || 16 * w.row_stride >= ((size_t)1 << 31))
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)((w.n_rows + 15) / 16), (unsigned)((t_rows + 15) / 16));
    if (w.dtype == T_Q4_0)
        hipLaunchKernelGGL(k_gemv_q8_mfma<true>, grid, dim3(64), 0, s, w, preq, (int)t_rows, out);
    else
        hipLaunchKernelGGL(k_gemv_q8_mfma<false>, grid, dim3(64), 0, s, w, preq, (int)t_rows, out);
    return hipGetLastError();
}

}  // namespace rce_qmm

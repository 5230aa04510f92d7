// gemv_q6_k.hip -- the Q6_K decode kernels (EXACT: one chain lane per row; Q8).
#include "gemv_chain_pipe.h"
#include "lds_limit.h"
#include "qmm_gemv_kernels.h"

namespace rce_qmm {
namespace {

// ---------------------------------------------------------------------------
// Q6_K EXACT: one lane per row (the row sum is a single chain); this form,
// which also forms its own products, serves rows longer than the LDS holds.
// ---------------------------------------------------------------------------

// rce-op-qmm/src/lib.rs L425-454, L1667-1705: per half o, l in 0..32, the
// positions l, l+32, l+64, l+96 in order: sumf += ((d sc) q) a.
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
#pragma unroll
                for (int m = 0; m < 4; m++)
#pragma unroll
                    for (int j = 0; j < 4; j++) x[m][j] = al[j + 32 * m];
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

// Rows longer than Q6_EXACT_LDS_K: the activations are read from global
// memory (each lane the same addresses) instead of LDS.
constexpr size_t Q6_EXACT_LDS_K = 16384;
__global__ __launch_bounds__(256) void k_gemv_exact_q6k(DevWeight w, const float *__restrict__ A,
                                                        float *__restrict__ out) {
    const size_t row = (size_t)blockIdx.x * 256 + threadIdx.x;
    // Lanes past the end recompute the last row (no branch around loads).
    const size_t rr = row < w.n_rows ? row : w.n_rows - 1;
    const int nsb = (int)(w.n_cols / 256);
    const float *a = A + (size_t)blockIdx.y * w.n_cols;
    float sumf = 0.0f;
    RawQ6_K b0, b1;
    ld_q6_k(w, rr, 0, b0);
    int sb = 0;
    for (; sb + 1 < nsb; sb += 2) {
        ld_q6_k(w, rr, sb + 1, b1);
        sumf = q6_exact_superblock(b0, a + 256 * sb, sumf);
        if (sb + 2 < nsb) ld_q6_k(w, rr, sb + 2, b0);
        sumf = q6_exact_superblock(b1, a + 256 * (sb + 1), sumf);
    }
    if (sb < nsb) sumf = q6_exact_superblock(b0, a + 256 * sb, sumf);
    if (row < w.n_rows) out[(size_t)blockIdx.y * w.n_rows + row] = sumf;
}

// The same row chains with the products formed by helper waves (the
// pipeline of gemv_chain_pipe.h), for k <= Q6_EXACT_LDS_K.  A block serves
// 64 rows of a group with four waves, one per SIMD: wave 0 holds the chains,
// waves 1..3 form the products (a fifth wave would share the chain's SIMD
// and the chain, which every barrier waits for, would get half its issue
// slots).  The unit of work is a pair: steps l = 8 p .. 8 p + 7, m = 0..3
// (positions 128 o + l + 32 m) of half o of a super-block, pairs numbered
// g = 8 sb + 4 o + p in the chain's order.  Stage s is pairs 3 s .. 3 s + 2,
// helper h forming pair 3 s + h - 1 from 8-byte slices of its ql, qh and
// scale chunks and the rows' d; pairs past the row give +0.0 products, which
// leave a chain (from +0.0, never -0.0) unchanged.
constexpr int Q6_DS = 8;  // stages of loads a helper keeps in flight

__global__ __launch_bounds__(256) void k_gemv_exact_q6k_split(DevWeight w, const float *__restrict__ A,
                                                              float *__restrict__ out) {
    constexpr int SV = 96;  // chain steps per stage: 3 pairs
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const size_t t = blockIdx.y, row0 = (size_t)blockIdx.x * 64;
    const size_t k = w.n_cols;
    const int np = (int)(k / 256) * 8;  // pairs in a row
    const int ns = (np + 2) / 3;
    const int s_tot = (ns + Q6_DS - 1) / Q6_DS * Q6_DS;
    extern __shared__ __align__(16) unsigned char lds[];
    float *act = reinterpret_cast<float *>(lds);  // k values, then a 16-byte dump slot
    float4 *prod = reinterpret_cast<float4 *>(act + k + 4);  // [2][24][64]
    const int hw = wv - 1;
    const uint8_t *gb = w.base + (row0 / 64) * w.group_stride;
    const WBuf wq = make_wbuf(gb, (uint32_t)lane * 16);  // chunk slices
    const WBuf wd = make_wbuf(gb, (uint32_t)lane * 2);   // d
    struct Slice { uint2 qa, qb, qh, sc; uint32_t d; };
    // pair g's slices (g past the row: the last pair's, not used)
    auto load = [&](int s, Slice &v) {
        const int g = min(3 * s + hw, np - 1), o = (g >> 2) & 1, p = g & 3, c = p >> 1;
        const uint32_t so = (uint32_t)(g >> 3) * (uint32_t)IL64_Q6K_SB, b8 = 8u * (uint32_t)(p & 1);
        v.qa = bld8(wq, (uint32_t)(4 * o + c) * 1024u + b8, so);
        v.qb = bld8(wq, (uint32_t)(4 * o + 2 + c) * 1024u + b8, so);
        v.qh = bld8(wq, (uint32_t)(8 + 2 * o + c) * 1024u + b8, so);
        v.sc = bld8(wq, 12u * 1024u + 8u * (uint32_t)o, so);
        v.d = bld2(wd, (uint32_t)IL64_Q6K_D, so);
    };
    Slice ring[Q6_DS];
    if (wv != 0) {
#pragma unroll
        for (int j = 0; j < Q6_DS; j++) load(j, ring[j]);
    }
    stage_act<256, 16>(A + t * k, k, k, act, [](size_t i) { return i; });
    __syncthreads();
    if (wv == 0) {
        const float acc = run_chain<SV, 64>(prod + lane, ns, s_tot);
        const size_t row = row0 + lane;
        if (row < w.n_rows) out[t * w.n_rows + row] = acc;
        return;
    }
    // the pair's 32 activations (positions 8 p + 4 h + 32 m .. + 3 of its
    // half, h = 0, 1), read during the stage before
    float4 an[2][2][4];
    auto read_act = [&](int s, float4 (*dst)[4]) {
        const int g = min(3 * s + hw, np - 1);
        const float *ah = act + (size_t)(g >> 3) * 256 + 128 * ((g >> 2) & 1) + 8 * (g & 3);
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int m = 0; m < 4; m++) dst[h][m] = *reinterpret_cast<const float4 *>(ah + 4 * h + 32 * m);
    };
    read_act(0, an[0]);
    for (int s0 = 0; s0 < s_tot; s0 += Q6_DS) {
#pragma unroll
        for (int u = 0; u < Q6_DS; u++) {
            const int s = s0 + u;
            read_act(s + 1, an[(u + 1) & 1]);
            const Slice v = ring[u];
            const int g = 3 * s + hw, c = (g & 3) >> 1;
            // (d sc) per m as the reference forms it, and -32 (d sc) for the
            // fma that rounds (q - 32) (d sc) once
            const float d = h2f(v.d);
            float ds[4], nn[4];
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const int bi = c + 2 * m;  // scale byte 8 o + is + 2 m within the half's 8 bytes
                const uint32_t wsc = (bi >> 2) ? v.sc.y : v.sc.x;
                ds[m] = d * (float)(int)(int8_t)((wsc >> (8 * (bi & 3))) & 0xFFu);
                nn[m] = -32.0f * ds[m];
            }
            float4 pr[2][4];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t qa = h ? v.qa.y : v.qa.x, qb = h ? v.qb.y : v.qb.x, qh = h ? v.qh.y : v.qh.x;
                const uint32_t uq[4] = {(qa & NIB) | ((qh & 0x03030303u) << 4), (qb & NIB) | ((qh & 0x0C0C0C0Cu) << 2),
                                        ((qa >> 4) & NIB) | (qh & 0x30303030u),
                                        ((qb >> 4) & NIB) | ((qh >> 2) & 0x30303030u)};
                float pj[4][4];  // [J][m]
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    const float4 x = an[u & 1][h][m];
                    const float xa[4] = {x.x, x.y, x.z, x.w};
                    pj[0][m] = __builtin_fmaf(ubyte<0>(uq[m]), ds[m], nn[m]) * xa[0];
                    pj[1][m] = __builtin_fmaf(ubyte<1>(uq[m]), ds[m], nn[m]) * xa[1];
                    pj[2][m] = __builtin_fmaf(ubyte<2>(uq[m]), ds[m], nn[m]) * xa[2];
                    pj[3][m] = __builtin_fmaf(ubyte<3>(uq[m]), ds[m], nn[m]) * xa[3];
                }
#pragma unroll
                for (int j = 0; j < 4; j++) pr[h][j] = make_float4(pj[j][0], pj[j][1], pj[j][2], pj[j][3]);
            }
            load(s + Q6_DS, ring[u]);  // the slot's next stage once this one is used
            float4 *pp = prod + ((size_t)(s & 1) * (SV / 4) + 8 * hw) * 64 + lane;
            if (g < np) {
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int j = 0; j < 4; j++) pp[(size_t)(4 * h + j) * 64] = pr[h][j];
            } else {  // past the row: +0.0 steps
#pragma unroll
                for (int j = 0; j < 8; j++) pp[(size_t)j * 64] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
            __syncthreads();
        }
    }
}

hipError_t launch_q6_split(const DevWeight &w, const float *a, size_t t_rows, float *out, hipStream_t s) {
    const size_t lds = (w.n_cols + 4) * sizeof(float) + 2 * 96 * 64 * sizeof(float);
    if (lds > 64 * 1024) {  // activations of a long row: more than the default 64 KB
        const hipError_t e = ensure_lds_limit((const void *)k_gemv_exact_q6k_split, 160 * 1024);
        if (e != hipSuccess) return e;
    }
    const dim3 grid((unsigned)((w.n_rows + 63) / 64), (unsigned)t_rows);
    hipLaunchKernelGGL(k_gemv_exact_q6k_split, grid, dim3(256), lds, s, w, a, out);
    return hipGetLastError();
}

}  // namespace

hipError_t q6_prepare_lds() { return ensure_lds_limit((const void *)k_gemv_exact_q6k_split, 160 * 1024); }

hipError_t launch_gemv_q6_k(const DevWeight &w, const GemvGeom &g, const float *a, size_t t_rows, float *out, int mode,
                            hipStream_t s) {
    if (mode == 0) {
        if (w.n_cols <= Q6_EXACT_LDS_K) return launch_q6_split(w, a, t_rows, out, s);
        dim3 grid((unsigned)((w.n_rows + 255) / 256), (unsigned)t_rows);
        hipLaunchKernelGGL(k_gemv_exact_q6k, grid, dim3(256), 0, s, w, a, out);
        return hipGetLastError();
    }
    return launch_as_tb<Q6_KQ8, true, 2>(w, g, a, t_rows, out, s);
}
hipError_t launch_gemv_fx_q6_k(const FxLaunch &f, const GemvGeom &g, const float *a, int mode, hipStream_t s) {
    if (mode == 0) return hipErrorInvalidValue;  // EXACT Q6_K is one lane per row
    return launch_as_fx_nt<Q6_KQ8<1>, true>(f, g, a, s);
}
}  // namespace rce_qmm

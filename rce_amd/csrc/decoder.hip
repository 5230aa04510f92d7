// decoder.hip -- the non-linear steps of the Llama-2 decode step that sit
// between the quantized matmuls (rce-tinyllama/src/lib.rs L158-330 with
// rce-op-attn/src/lib.rs L107-251), so that activations stay in HBM for the
// whole token.  The matmuls themselves are the decode GEMV kernels
// (qmm_gemv_kernels.h), in their fused forms where the step allows.
//
// Numerics (each kernel states its own):
//   * rms_norm: the sum of squares is a fixed-shape tree (run-to-run
//     deterministic) where the reference folds sequentially, so the norm's
//     scale may differ from the reference's in the last bits; every other
//     operation is the reference's, one rounding each.
//   * RoPE: the (cos, sin) table is built on the host with the C library's
//     logf / expf / sinf / cosf in the reference's expression order (the
//     functions Rust's f32 methods call on Linux), so the rotation is the
//     reference's bit for bit.
//   * attention: the reference's softmax-weighted sum of the values,
//     evaluated with fixed-shape parallel reductions instead of its
//     key-by-key recurrence (f32 reassociation; one key gives v exactly);
//     exp is the library's rce_exp (last-bit differences from the host libm).
//   * silu: silu_ref (rce_exp).
// This file is built with -ffp-contract=off: no multiply-add contraction.
#include "qmm_internal.h"

namespace rce_qmm {
namespace {

constexpr int NORM_NT = 256;

__device__ __forceinline__ float wave_sum(float v) {
    // fixed butterfly: the same tree on every call
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off);
    return v;
}

// rce-tinyllama/src/lib.rs L158-163: mean_sq = sum(v*v) / n,
// inv = 1 / sqrt(mean_sq + eps), out = (v * inv) * w.
__global__ __launch_bounds__(NORM_NT) void k_rms_norm(const float *__restrict__ x, const float *__restrict__ w, int n,
                                                      float eps, float *__restrict__ out, int *pos, int ctx_len,
                                                      int *status) {
    __shared__ float part[NORM_NT / 64];
    const int t = threadIdx.x;
    if (pos && t == 0 && status[2] == 0) {  // the last norm of a decode step advances the position
        const int p = pos[0];
        if (p >= ctx_len && status[0] == 0) status[0] = 2;
        pos[0] = p + 1;
    }
    float ss = 0.0f;
    for (int i = t; i < n; i += NORM_NT) {
        const float sq = x[i] * x[i];
        ss = ss + sq;
    }
    ss = wave_sum(ss);
    if ((t & 63) == 0) part[t >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < NORM_NT / 64; i++) tot = tot + part[i];
    const float mean_sq = tot / (float)n;
    const float inv = 1.0f / sqrtf(mean_sq + eps);
    for (int i = t; i < n; i += NORM_NT) {
        const float v = x[i] * inv;
        out[i] = v * w[i];
    }
}

// Attention of one decode step: one block of NW waves per query head h;
// kv head g = h / (n_q / n_kv) (rce-tinyllama L262-281).
//  1. The block loads this position's q_h, k_g, v_g into LDS (issued before
//     the position is read: they do not depend on it), then the RoPE row,
//     and rotates q_h and k_g (rce-op-attn L115-151): pairs (i, i + half) ->
//     (a c - b s, a s + b c).  The block of the first query head of each kv
//     group appends k_g, v_g to the caches (every block uses its own copy of
//     this position's k and v, so no block waits for another).
//  2. Wave w takes the keys [w*seq/NW, (w+1)*seq/NW) in runs of CH (64 for
//     d_head 64, 32 for 128), all of a run's loads in flight together: lane
//     j scores key j (the reference's sequential dot, times scale); the
//     run's maximum and the sum of p_j = exp(s_j - m) are wave reductions
//     of fixed shape; out[d] = sum_j p_j v_j[d] as four partial sums over
//     the keys j = 0, 1, 2, 3 (mod 4), added (a0 + a1) + (a2 + a3).  A
//     wave's runs merge by rescaling with exp(m_old - m_new).
//  3. The waves' (m, l, out) merge in wave order through LDS (M = max m_w;
//     out = sum_w exp(m_w - M) out_w, l = sum_w exp(m_w - M) l_w), then
//     out *= 1 / l.
// This is the softmax-weighted sum that fused_attend_head_window
// (rce-op-attn L196-251) folds key by key with its online recurrence,
// evaluated in parallel: every reduction has a fixed shape (run-to-run
// bit-identical), and the result differs from the reference's by f32
// reassociation only (one key gives v exactly, as the reference's first
// key gives).
// Cache layouts (per layer): keys in tiles of 64 positions, [kv head]
// [position / 64][dimension / 4][position % 64][dimension % 4], so that a
// lane per key reads four dimensions of its key with one 16-byte load and
// a wave's load is one contiguous kilobyte (d_head / 4 loads per run);
// values [position][kv head][dimension], read as 16-byte quads by
// 64 / (d_head / 4) keys per load.  The caches hold ceil(ctx / 64) * 64
// positions.
// Waves per head: one per SIMD.  A run keeps a key row, its value quads
// and q in registers (about 200 for d_head 64), so the kernel asks for one
// wave per SIMD and the whole register file: a launch has n_q blocks at
// most.
constexpr int ATT_NW = 4;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

__device__ __forceinline__ float f4e(const float4 &v, int e) { return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w; }
__device__ __forceinline__ float &f4e(float4 &v, int e) { return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w; }

// Float offset of (position p, dimension d) in one kv head's key tiles.
template <int DH>
__device__ __forceinline__ size_t key_off(int p, int d) {
    return (size_t)(p >> 6) * (64 * DH) + (size_t)(d >> 2) * 256 + (size_t)(p & 63) * 4 + (d & 3);
}

template <int DH>
__global__ __launch_bounds__(64 * ATT_NW) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_attention(const float *__restrict__ qkv,
                                                           const float *__restrict__ rope_cs,
                                                           float *__restrict__ k_cache, float *__restrict__ v_cache,
                                                           const int *__restrict__ pos_p, int ctx_len, int n_q,
                                                           int n_kv, int rope_dim, float scale,
                                                           float *__restrict__ att, const int *__restrict__ skip) {
    constexpr int NQD = DH / 4;      // dimension quads of a key
    constexpr int KPI = 64 / NQD;    // keys per value load (4 or 2)
    constexpr int NA = 4 / KPI;      // partial sums a lane holds (1 or 2)
    constexpr int CH = 4096 / DH;    // keys per run (64 or 32)
    constexpr int VL = CH / KPI;     // value loads per run (16)
    __shared__ float qs[DH], ks[DH], vs[DH], cs[DH];
    __shared__ float mo[ATT_NW][DH + 2];  // each wave's out[DH], m, l
    // the wave index in a scalar register: the run bounds below are then
    // wave-uniform and their branches scalar
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), h = blockIdx.x;
    const int qpk = n_q / n_kv, g = h / qpk;
    const int kk = lane / NQD, dq = lane % NQD;  // value lanes: key kk of each KPI, dimensions 4 dq .. 4 dq + 3
    const size_t qd = (size_t)n_q * DH, kvd = (size_t)n_kv * DH, ctxp = ((size_t)ctx_len + 63) & ~(size_t)63;
    for (int i = tid; i < DH; i += 64 * ATT_NW) {  // independent of the position
        qs[i] = qkv[(size_t)h * DH + i];
        ks[i] = qkv[qd + (size_t)g * DH + i];
        vs[i] = qkv[qd + kvd + (size_t)g * DH + i];
    }
    // this position's value quad (not in the cache yet)
    const float4 vcur = *reinterpret_cast<const float4 *>(qkv + qd + kvd + (size_t)g * DH + 4 * dq);
    const int pos = pos_p[0];
    if (pos < 0 || pos >= ctx_len) return;  // the whole block; the step's last kernel reports it
    const int seq = pos + 1, half = rope_dim / 2;
    for (int i = tid; i < 2 * half; i += 64 * ATT_NW) cs[i] = rope_cs[(size_t)pos * half * 2 + i];
    const int j0 = (int)((long)wave * seq / ATT_NW), j1 = (int)((long)(wave + 1) * seq / ATT_NW);
    const float *kbase = k_cache + (size_t)g * DH * ctxp, *vbase = v_cache + (size_t)g * DH + 4 * dq;

    float4 kq[NQD];   // this lane's key, four dimensions per load
    float4 vv[VL];    // value quads of keys kk, kk + KPI, ... of the run
    // A run's cached keys / values, every load unconditional: rows at or
    // past pos read row 0 (always in range); key rows at or past pos are
    // unused (the current key comes from LDS).  The loaded value rows are
    // replaced where they are consumed: row pos by this
    // position's values, rows past pos by 0, so every value row used is
    // finite.  Doing that here instead would put a branch after each load
    // whose untaken side waits for the load, and the run's loads would no
    // longer be in flight together.
    auto load_run = [&](int c0) {
        const int r = c0 + lane;
        const float4 *kp = reinterpret_cast<const float4 *>(kbase + key_off<DH>(r < pos ? r : 0, 0));
#pragma unroll
        for (int i = 0; i < NQD; i++) kq[i] = kp[64 * i];
#pragma unroll
        for (int i = 0; i < VL; i++) {
            const int rj = c0 + i * KPI + kk;
            vv[i] = *reinterpret_cast<const float4 *>(vbase + (size_t)(rj < pos ? rj : 0) * kvd);
        }
    };
    if (j0 < j1) load_run(j0);
    __syncthreads();
    for (int i = tid; i < half; i += 64 * ATT_NW) {
        const float c = cs[2 * i], s = cs[2 * i + 1];
        float a = qs[i], b = qs[i + half];
        float ac = a * c, bs = b * s, as = a * s, bc = b * c;
        qs[i] = ac - bs;
        qs[i + half] = as + bc;
        a = ks[i];
        b = ks[i + half];
        ac = a * c; bs = b * s; as = a * s; bc = b * c;
        ks[i] = ac - bs;
        ks[i + half] = as + bc;
    }
    __syncthreads();
    if (h % qpk == 0 && wave == 0 && !(skip && skip[0])) {  // append this position to the layer's caches
        float *kd = k_cache + (size_t)g * DH * ctxp, *vd = v_cache + (size_t)pos * kvd + (size_t)g * DH;
#pragma unroll
        for (int d = 0; d < DH / 64; d++) {
            kd[key_off<DH>(pos, lane + 64 * d)] = ks[lane + 64 * d];
            vd[lane + 64 * d] = vs[lane + 64 * d];
        }
    }
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);  // out[4 dq .. 4 dq + 3]
    float m = -INFINITY, l = 0.0f;
    if (j0 < j1) {
        float q[DH];  // every lane needs all of q for its key's dot
#pragma unroll
        for (int i = 0; i < DH; i++) q[i] = qs[i];
        for (int c0 = j0; c0 < j1; c0 += CH) {
            const int n = min(CH, j1 - c0);
            if (c0 > j0) load_run(c0);
            if (c0 + lane == pos) {  // this lane's key is the current position
#pragma unroll
                for (int i = 0; i < NQD; i++) kq[i] = make_float4(ks[4 * i], ks[4 * i + 1], ks[4 * i + 2], ks[4 * i + 3]);
            }
            float sc = -INFINITY;
            if (lane < n) {
                float dot = 0.0f;
#pragma unroll
                for (int d = 0; d < DH; d++) {
                    const float pr = q[d] * f4e(kq[d >> 2], d & 3);
                    dot = dot + pr;
                }
                sc = dot * scale;
            }
            const float m_new = fmaxf(m, wave_max(sc));  // finite: the run has a key
            const float corr = rce_exp(m - m_new);           // 0 for the wave's first run
            const float p = lane < n ? rce_exp(sc - m_new) : 0.0f;
            const float lc = l * corr;
            l = lc + wave_sum(p);
            // a[i % NA] sums the keys i KPI + kk: partial sum (i KPI + kk) % 4
            float4 a[NA];
#pragma unroll
            for (int s = 0; s < NA; s++) a[s] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            // p = 0 and finite value rows past the run's keys: whole loads of
            // KPI keys.  A constant trip count with a uniform test per load
            // (not a break), so the loop unrolls and vv stays in registers.
#pragma unroll
            for (int i = 0; i < VL; i++) {
                if (i * KPI >= n) continue;
                const int rj = c0 + i * KPI + kk;
                const float pj = __shfl(p, i * KPI + kk);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float v = rj < pos ? f4e(vv[i], e) : (rj == pos ? f4e(vcur, e) : 0.0f);
                    const float t = pj * v;
                    f4e(a[i % NA], e) = f4e(a[i % NA], e) + t;
                }
            }
            // (a0 + a1) + (a2 + a3): with KPI 4 lane group kk holds a_kk; with
            // KPI 2 group kk holds a_kk and a_(kk + 2)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float sv;
                if constexpr (NA == 1) {
                    const float x = f4e(a[0], e);
                    const float s = x + __shfl_xor(x, 16);
                    sv = s + __shfl_xor(s, 32);
                } else {
                    const float x0 = f4e(a[0], e), x1 = f4e(a[1], e);
                    const float s01 = x0 + __shfl_xor(x0, 32), s23 = x1 + __shfl_xor(x1, 32);
                    sv = s01 + s23;
                }
                const float oc = f4e(o, e) * corr;
                f4e(o, e) = oc + sv;
            }
            m = m_new;
        }
    }
    float *out = att + (size_t)h * DH;
    if (kk == 0) *reinterpret_cast<float4 *>(&mo[wave][4 * dq]) = o;
    if (lane == 0) {
        mo[wave][DH] = m;  // -inf: a wave without keys
        mo[wave][DH + 1] = l;
    }
    __syncthreads();
    if (wave != 0) return;
    constexpr int DPL = DH / 64;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < ATT_NW; w++) M = fmaxf(M, mo[w][DH]);
    float acc[DPL], lacc = 0.0f;
#pragma unroll
    for (int d = 0; d < DPL; d++) acc[d] = 0.0f;
#pragma unroll
    for (int w = 0; w < ATT_NW; w++) {
        if (mo[w][DH] == -INFINITY) continue;  // a wave without keys
        const float wt = rce_exp(mo[w][DH] - M);
#pragma unroll
        for (int d = 0; d < DPL; d++) {
            const float t = wt * mo[w][lane + 64 * d];
            acc[d] = acc[d] + t;
        }
        const float lw = wt * mo[w][DH + 1];
        lacc = lacc + lw;
    }
    const float inv = 1.0f / lacc;
#pragma unroll
    for (int d = 0; d < DPL; d++) out[lane + 64 * d] = acc[d] * inv;
}

__global__ void k_swiglu(const float *__restrict__ g, const float *__restrict__ u, float *__restrict__ h, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) h[i] = silu_ref(g[i]) * u[i];  // rce-tinyllama L320
}

__global__ void k_add_inplace(float *__restrict__ x, const float *__restrict__ o, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = x[i] + o[i];  // rce-tinyllama L318, L323
}

}  // namespace

hipError_t launch_rms_norm(const float *x, const float *w, size_t n, float eps, float *out, int *pos, int ctx_len,
                           int *status, hipStream_t s) {
    hipLaunchKernelGGL(k_rms_norm, dim3(1), dim3(NORM_NT), 0, s, x, w, (int)n, eps, out, pos, ctx_len, status);
    return hipGetLastError();
}

bool attention_supports(int d_head, int rope_dim) {
    return (d_head == 64 || d_head == 128) && rope_dim >= 0 && rope_dim <= d_head && rope_dim % 2 == 0;
}

hipError_t launch_attention(const float *qkv, const float *rope_cs, float *k_cache, float *v_cache, const int *pos,
                            int ctx_len, int n_q, int n_kv, int d_head, int rope_dim, float scale, float *att,
                            const int *skip, hipStream_t s) {
    if (n_kv <= 0 || n_q % n_kv) return hipErrorInvalidValue;
    switch (d_head) {
    case 64:
        hipLaunchKernelGGL(k_attention<64>, dim3(n_q), dim3(64 * ATT_NW), 0, s, qkv, rope_cs, k_cache, v_cache, pos,
                           ctx_len, n_q, n_kv, rope_dim, scale, att, skip);
        break;
    case 128:
        hipLaunchKernelGGL(k_attention<128>, dim3(n_q), dim3(64 * ATT_NW), 0, s, qkv, rope_cs, k_cache, v_cache, pos,
                           ctx_len, n_q, n_kv, rope_dim, scale, att, skip);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_swiglu(const float *g, const float *u, float *h, size_t n, hipStream_t s) {
    hipLaunchKernelGGL(k_swiglu, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, g, u, h, n);
    return hipGetLastError();
}

hipError_t launch_add_inplace(float *x, const float *o, size_t n, hipStream_t s) {
    hipLaunchKernelGGL(k_add_inplace, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, o, n);
    return hipGetLastError();
}

}  // namespace rce_qmm

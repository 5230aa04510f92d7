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
//     j scores key j (the reference's sequential dot, times scale; the key
//     cache is transposed, [kv head][dimension][position], so each dimension
//     of a run is one coalesced load instead of one cache line per key); the
//     run's maximum and the sum of p_j = exp(s_j - m) are wave reductions
//     of fixed shape; out[d] = sum_j p_j v_j[d] (lane = d, four partial sums
//     added in a fixed order).  A wave's runs merge by rescaling with
//     exp(m_old - m_new).
//  3. The waves' (m, l, out) merge in wave order through LDS (M = max m_w;
//     out = sum_w exp(m_w - M) out_w, l = sum_w exp(m_w - M) l_w), then
//     out *= 1 / l.
// This is the softmax-weighted sum that fused_attend_head_window
// (rce-op-attn L196-251) folds key by key with its online recurrence,
// evaluated in parallel: every reduction has a fixed shape (run-to-run
// bit-identical), and the result differs from the reference's by f32
// reassociation only (one key: out = v exactly, as the reference's first
// key gives).
// Waves per head: one per SIMD.  A run keeps a key row, a value column and
// q in registers (about 200 for d_head 64), so the kernel asks for one wave
// per SIMD and the whole register file: a launch has n_q blocks at most.
constexpr int ATT_NW = 4;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

template <int DH>
__global__ __launch_bounds__(64 * ATT_NW) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_attention(const float *__restrict__ qkv,
                                                           const float *__restrict__ rope_cs,
                                                           float *__restrict__ k_cache, float *__restrict__ v_cache,
                                                           const int *__restrict__ pos_p, int ctx_len, int n_q,
                                                           int n_kv, int rope_dim, float scale,
                                                           float *__restrict__ att, const int *__restrict__ skip) {
    constexpr int DPL = DH / 64;    // dimensions per lane
    constexpr int CH = 4096 / DH;   // keys per run (64 or 32)
    __shared__ float qs[DH], ks[DH], vs[DH], cs[DH];
    __shared__ float mo[ATT_NW][DH + 2];  // each wave's out[DH], m, l
    // the wave index in a scalar register: the run bounds below are then
    // wave-uniform and their branches scalar
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), h = blockIdx.x;
    const int qpk = n_q / n_kv, g = h / qpk;
    const size_t qd = (size_t)n_q * DH, kvd = (size_t)n_kv * DH;
    for (int i = tid; i < DH; i += 64 * ATT_NW) {  // independent of the position
        qs[i] = qkv[(size_t)h * DH + i];
        ks[i] = qkv[qd + (size_t)g * DH + i];
        vs[i] = qkv[qd + kvd + (size_t)g * DH + i];
    }
    const int pos = pos_p[0];
    if (pos < 0 || pos >= ctx_len) return;  // the whole block; the step's last kernel reports it
    const int seq = pos + 1, half = rope_dim / 2;
    for (int i = tid; i < 2 * half; i += 64 * ATT_NW) cs[i] = rope_cs[(size_t)pos * half * 2 + i];
    const int j0 = (int)((long)wave * seq / ATT_NW), j1 = (int)((long)(wave + 1) * seq / ATT_NW);
    // keys are stored transposed, [kv head][dimension][position], so that a
    // lane per key reads each dimension of a run with one coalesced load
    const float *kbase = k_cache + (size_t)g * DH * ctx_len, *vbase = v_cache + (size_t)g * DH;

    float kt[DH];
    float vv[CH][DPL];
    float vcur[DPL];  // this position's value column (not in the cache yet)
#pragma unroll
    for (int d = 0; d < DPL; d++) vcur[d] = qkv[qd + kvd + (size_t)g * DH + lane + 64 * d];
    // A run's cached keys / values, every load unconditional: rows at or
    // past pos read row 0 (always in range); key rows at or past pos are
    // unused (the current key comes from LDS).  The loaded value rows are
    // replaced where they are consumed (value_at): row pos by this
    // position's values, rows past pos by 0, so every value row used is
    // finite.  Doing that here instead would put a branch after each load
    // whose untaken side waits for the load, and the run's loads would no
    // longer be in flight together.
    auto load_run = [&](int c0) {
        const int r = c0 + lane;
        const float *kp = kbase + (r < pos ? r : 0);
#pragma unroll
        for (int d = 0; d < DH; d++) kt[d] = kp[(size_t)d * ctx_len];
#pragma unroll
        for (int j = 0; j < CH; j++) {
            const int rj = c0 + j;
            const float *vp = vbase + (size_t)(rj < pos ? rj : 0) * kvd;
#pragma unroll
            for (int d = 0; d < DPL; d++) vv[j][d] = vp[lane + 64 * d];
        }
    };
    auto value_at = [&](int rj, int j, int d) {
        return rj < pos ? vv[j][d] : (rj == pos ? vcur[d] : 0.0f);
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
        float *kd = k_cache + (size_t)g * DH * ctx_len + pos, *vd = v_cache + (size_t)pos * kvd + (size_t)g * DH;
#pragma unroll
        for (int d = 0; d < DPL; d++) {
            kd[(size_t)(lane + 64 * d) * ctx_len] = ks[lane + 64 * d];
            vd[lane + 64 * d] = vs[lane + 64 * d];
        }
    }
    float o[DPL];
#pragma unroll
    for (int d = 0; d < DPL; d++) o[d] = 0.0f;
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
                for (int d = 0; d < DH; d++) kt[d] = ks[d];
            }
            float sc = -INFINITY;
            if (lane < n) {
                float dot = 0.0f;
#pragma unroll
                for (int d = 0; d < DH; d++) {
                    const float pr = q[d] * kt[d];
                    dot = dot + pr;
                }
                sc = dot * scale;
            }
            const float m_new = fmaxf(m, wave_max(sc));  // finite: the run has a key
            const float corr = rce_exp(m - m_new);           // 0 for the wave's first run
            const float p = lane < n ? rce_exp(sc - m_new) : 0.0f;
            const float lc = l * corr;
            l = lc + wave_sum(p);
            float a[4][DPL];
#pragma unroll
            for (int k = 0; k < 4; k++)
#pragma unroll
                for (int d = 0; d < DPL; d++) a[k][d] = 0.0f;
            // p = 0 and finite value rows past the run's keys: whole groups of
            // four.  A constant trip count with a uniform test per group (not
            // a break), so the loop unrolls and vv stays in registers.
#pragma unroll
            for (int j = 0; j < CH; j += 4) {
                if (j >= n) continue;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float pj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), j + k));
#pragma unroll
                    for (int d = 0; d < DPL; d++) {
                        const float t = pj * value_at(c0 + j + k, j + k, d);
                        a[k][d] = a[k][d] + t;
                    }
                }
            }
#pragma unroll
            for (int d = 0; d < DPL; d++) {
                const float s01 = a[0][d] + a[1][d], s23 = a[2][d] + a[3][d];
                const float sv = s01 + s23, oc = o[d] * corr;
                o[d] = oc + sv;
            }
            m = m_new;
        }
    }
    float *out = att + (size_t)h * DH;
#pragma unroll
    for (int d = 0; d < DPL; d++) mo[wave][lane + 64 * d] = o[d];
    if (lane == 0) {
        mo[wave][DH] = m;  // -inf: a wave without keys
        mo[wave][DH + 1] = l;
    }
    __syncthreads();
    if (wave != 0) return;
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

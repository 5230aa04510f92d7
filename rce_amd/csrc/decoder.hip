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
//   * attention: the reference's key order and recurrence; exp is the
//     device's expf (last-bit differences from the host libm).
//   * silu: silu_ref (device expf).
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
    if (pos && t == 0) {  // the last norm of a decode step advances the position
        const int p = pos[0];
        if (p >= ctx_len) status[0] = 2;
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

// One block (one wave) per query head h; kv head g = h / (n_q / n_kv)
// (rce-tinyllama L262-281).  Steps:
//  1. q_h and k_g, v_g of this position from the q|k|v projections;
//     RoPE of q_h and k_g (rce-op-attn L115-151): pairs (i, i + half),
//     (a, b) -> (a c - b s, a s + b c) with the position's table row.
//  2. The first query head of each kv group appends k_g, v_g to the caches
//     at pos (every head of the group uses its own copy of this position's
//     k and v, so no block waits for another).
//  3. fused_attend_head_window (rce-op-attn L196-251) over keys 0..pos in
//     order: s_j = dot(q, k_j) * scale (dot: sequential sum of products);
//     key 0 sets out = 0 + 1 * v_0, l = 1; key j > 0: m' = max(m, s_j),
//     alpha = exp(m - m'), beta = exp(s_j - m'), out = out * alpha +
//     beta * v_j, l = l * alpha + beta; finally out *= 1 / l.  Keys are
//     taken in chunks of CH: lane j loads key row j of the chunk and computes
//     s_j, every lane loads its dimensions of the chunk's value rows (all
//     loads of a chunk are issued together), the running maxima come from a
//     prefix max over the chunk (max is exact, so these equal the
//     reference's sequential maxima), and the out / l recurrence runs in key
//     order with lane = dimension.
template <int DH>
__global__ __launch_bounds__(64) void k_attention(const float *__restrict__ qkv, const float *__restrict__ rope_cs,
                                                  float *__restrict__ k_cache, float *__restrict__ v_cache,
                                                  const int *__restrict__ pos_p, int ctx_len, int n_q, int n_kv,
                                                  int rope_dim, float scale, float *__restrict__ att) {
    constexpr int DPL = DH / 64;    // dimensions per lane
    constexpr int CH = 4096 / DH;   // keys per chunk (64 or 32)
    constexpr int R4 = DH / 4;      // float4 pieces of a row
    __shared__ float qs[DH], ks[DH], cs[DH];
    const int lane = threadIdx.x, h = blockIdx.x;
    const int pos = pos_p[0];
    if (pos < 0 || pos >= ctx_len) return;  // the step's last kernel reports it
    const int qpk = n_q / n_kv, g = h / qpk;
    const size_t qd = (size_t)n_q * DH, kvd = (size_t)n_kv * DH;
    const int half = rope_dim / 2;
    const float *kbase = k_cache + (size_t)g * DH, *vbase = v_cache + (size_t)g * DH;

    // One round of loads: this position's q, k, v, the RoPE row, and the
    // first chunk of cached keys / values.  Cache rows at or past pos read
    // row 0 (always in range) and are replaced or unused, so every load is
    // unconditional and all are in flight together.
    float qr[DPL], kr[DPL], vcur[DPL], csr[DPL];
#pragma unroll
    for (int d = 0; d < DPL; d++) {
        const int i = lane + 64 * d;
        qr[d] = qkv[(size_t)h * DH + i];
        kr[d] = qkv[qd + (size_t)g * DH + i];
        vcur[d] = qkv[qd + kvd + (size_t)g * DH + i];
        csr[d] = i < 2 * half ? rope_cs[(size_t)pos * half * 2 + i] : 0.0f;
    }
    float4 kv[R4];
    float vv[CH][DPL];
    auto load_chunk = [&](int c0) {
        const int r = c0 + lane;
        const float4 *kp = reinterpret_cast<const float4 *>(kbase + (size_t)(r < pos ? r : 0) * kvd);
#pragma unroll
        for (int i = 0; i < R4; i++) kv[i] = kp[i];
#pragma unroll
        for (int j = 0; j < CH; j++) {
            const int rj = c0 + j;
            const float *vp = vbase + (size_t)(rj < pos ? rj : 0) * kvd;
#pragma unroll
            for (int d = 0; d < DPL; d++) vv[j][d] = vp[lane + 64 * d];
        }
    };
    load_chunk(0);
#pragma unroll
    for (int d = 0; d < DPL; d++) {
        qs[lane + 64 * d] = qr[d];
        ks[lane + 64 * d] = kr[d];
        cs[lane + 64 * d] = csr[d];
    }
    __syncthreads();
    // RoPE (rce-op-attn L115-151): pairs (i, i + half) -> (a c - b s, a s + b c)
    for (int i = lane; i < half; i += 64) {
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
    if (h % qpk == 0) {  // append this position to the layer's caches
        float *kd = k_cache + (size_t)pos * kvd + (size_t)g * DH, *vd = v_cache + (size_t)pos * kvd + (size_t)g * DH;
#pragma unroll
        for (int d = 0; d < DPL; d++) {
            kd[lane + 64 * d] = ks[lane + 64 * d];
            vd[lane + 64 * d] = vcur[d];
        }
    }
    // q in registers (every lane needs all of it for its key's dot)
    float q[DH];
#pragma unroll
    for (int i = 0; i < DH; i++) q[i] = qs[i];
    const int seq = pos + 1;
    float o[DPL];
#pragma unroll
    for (int d = 0; d < DPL; d++) o[d] = 0.0f;
    float m = -INFINITY, l = 0.0f;
    for (int c0 = 0; c0 < seq; c0 += CH) {
        if (c0 > 0) load_chunk(c0);
        const int n = min(CH, seq - c0);
        if (c0 + lane == pos) {  // this lane's key is the current position
#pragma unroll
            for (int i = 0; i < R4; i++) kv[i] = make_float4(ks[4 * i], ks[4 * i + 1], ks[4 * i + 2], ks[4 * i + 3]);
        }
        if (pos - c0 < CH) {  // the chunk holds the current position: its value row
            const int jp = pos - c0;
#pragma unroll
            for (int j = 0; j < CH; j++)
                if (j == jp) {
#pragma unroll
                    for (int d = 0; d < DPL; d++) vv[j][d] = vcur[d];
                }
        }
        float sc = -INFINITY;
        if (lane < n) {
            float dot = 0.0f;
#pragma unroll
            for (int i = 0; i < R4; i++) {
                float pr = q[4 * i] * kv[i].x;
                dot = dot + pr;
                pr = q[4 * i + 1] * kv[i].y;
                dot = dot + pr;
                pr = q[4 * i + 2] * kv[i].z;
                dot = dot + pr;
                pr = q[4 * i + 3] * kv[i].w;
                dot = dot + pr;
            }
            sc = dot * scale;
        }
        // running maxima: inclusive prefix max over the chunk, after m
        // (lanes past n hold -inf and come after every valid lane)
        float pm = sc;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float t = __shfl_up(pm, off);
            if (lane >= off) pm = fmaxf(pm, t);
        }
        const float m_incl = fmaxf(m, pm);
        float m_prev = __shfl_up(m_incl, 1);
        if (lane == 0) m_prev = m;
        const float alpha = lane < n ? expf(m_prev - m_incl) : 1.0f;
        const float beta = lane < n ? expf(sc - m_incl) : 0.0f;
        m = __shfl(m_incl, n - 1);
        // the recurrence in key order; key j's factors broadcast from lane j
#pragma unroll
        for (int j = 0; j < CH; j++) {
            if (j < n) {
                const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), j));
                const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, beta), j));
                if (c0 + j == 0) {  // the first key: out = 0 + 1 * v, l = 1
#pragma unroll
                    for (int d = 0; d < DPL; d++) {
                        const float t = 1.0f * vv[j][d];
                        o[d] = o[d] + t;
                    }
                    l = 1.0f;
                } else {
#pragma unroll
                    for (int d = 0; d < DPL; d++) {
                        const float t1 = o[d] * a, t2 = b * vv[j][d];
                        o[d] = t1 + t2;
                    }
                    const float la = l * a;
                    l = la + b;
                }
            }
        }
    }
    float *out = att + (size_t)h * DH;
    if (l != 0.0f) {
        const float inv = 1.0f / l;
#pragma unroll
        for (int d = 0; d < DPL; d++) o[d] = o[d] * inv;
    }
#pragma unroll
    for (int d = 0; d < DPL; d++) out[lane + 64 * d] = o[d];
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
                            hipStream_t s) {
    if (n_kv <= 0 || n_q % n_kv) return hipErrorInvalidValue;
    switch (d_head) {
    case 64:
        hipLaunchKernelGGL(k_attention<64>, dim3(n_q), dim3(64), 0, s, qkv, rope_cs, k_cache, v_cache, pos, ctx_len,
                           n_q, n_kv, rope_dim, scale, att);
        break;
    case 128:
        hipLaunchKernelGGL(k_attention<128>, dim3(n_q), dim3(64), 0, s, qkv, rope_cs, k_cache, v_cache, pos,
                           ctx_len, n_q, n_kv, rope_dim, scale, att);
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

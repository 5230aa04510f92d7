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
//  1. Every wave loads this position's q_h, k_g (and v_g) with element
//     lane + 64 d in lane `lane` (issued before the position is read: they
//     do not depend on it), then the RoPE row and the cache rows of its first
//     run, and rotates q and k in registers while those loads are in flight
//     (rce-op-attn L115-151): pairs (i, i + half) -> (a c - b s, a s + b c),
//     the partner element from its lane by a lane exchange.  Every lane then
//     reads all of q from the wave's own LDS row.  The wave whose last run
//     holds the current position forms that key's score,
//     the reference's sequential dot of q and the rotated k, from the
//     lanes' products, also while its loads are in flight.  The first wave
//     of the first query head of each kv group appends k_g, v_g to the
//     caches (every block uses its own copy of this position's k and v, so
//     no block waits for another).
//  2. Wave w takes the runs w, w + NW, w + 2 NW, ... of CH keys (64 for
//     d_head 64, 32 for 128; a wave loads whole runs, so at short contexts
//     one wave does the work of a block and the others leave at once), all
//     of a run's loads in flight together: lane j scores key j (the
//     reference's sequential dot, times scale); the run's maximum and the
//     sum of p_j = exp(s_j - m) are wave reductions of fixed shape;
//     out[d] = sum_j p_j v_j[d] as four partial sums over the keys j = 0,
//     1, 2, 3 (mod 4), added (a0 + a1) + (a2 + a3).  A wave's runs merge by
//     rescaling with exp(m_old - m_new).
//  3. The waves' (m, l, out) merge in wave order through LDS (M = max m_w;
//     out = sum_w exp(m_w - M) out_w, l = sum_w exp(m_w - M) l_w), then
//     out *= 1 / l: the block's only barrier.
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
// Waves per head: one per SIMD (a run keeps a key row and its value quads
// in registers), so a launch has n_q blocks at most.
constexpr int ATT_NW = 4;

// x + (x of lane ^ 16), x + (x of lane ^ 32), through the gfx950 row swaps
// (no LDS): with both operands x, permlane16_swap returns in its two
// halves, for every lane, its own x and the x of lane ^ 16 (in one order or
// the other), and permlane32_swap the same for lane ^ 32, so their sum is
// the pair's sum in every lane.
__device__ __forceinline__ float xor16_sum(float x) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}
__device__ __forceinline__ float xor32_sum(float x) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}

__device__ __forceinline__ float f4e(const float4 &v, int e) { return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w; }
__device__ __forceinline__ float &f4e(float4 &v, int e) { return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w; }

// x of lane l (every lane active)
__device__ __forceinline__ float lane_val(float x, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(l << 2, __builtin_bit_cast(int, x)));
}

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
    constexpr int DPL = DH / 64;     // elements per lane of q, k, v and out
    constexpr int NQD = DH / 4;      // dimension quads of a key
    constexpr int KPI = 64 / NQD;    // keys per value load (4 or 2)
    constexpr int NA = 4 / KPI;      // partial sums a lane holds (1 or 2)
    constexpr int CH = 4096 / DH;    // keys per run (64 or 32)
    constexpr int VL = CH / KPI;     // value loads per run (16)
    __shared__ float mo[ATT_NW][DH + 2];  // each wave's out[DH], m, l
    __shared__ float qw[ATT_NW][DH], pw[ATT_NW][DH];  // each wave's q and products q_i k_i
    // the wave index in a scalar register: the run bounds below are then
    // wave-uniform and their branches scalar
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), h = blockIdx.x;
    const int qpk = n_q / n_kv, g = h / qpk;
    const int kk = lane / NQD, dq = lane % NQD;  // value lanes: key kk of each KPI, dimensions 4 dq .. 4 dq + 3
    const size_t qd = (size_t)n_q * DH, kvd = (size_t)n_kv * DH, ctxp = ((size_t)ctx_len + 63) & ~(size_t)63;
    float qx[DPL], kx[DPL], vx[DPL];
#pragma unroll
    for (int d = 0; d < DPL; d++) {
        qx[d] = qkv[(size_t)h * DH + lane + 64 * d];
        kx[d] = qkv[qd + (size_t)g * DH + lane + 64 * d];
        vx[d] = qkv[qd + kvd + (size_t)g * DH + lane + 64 * d];
    }
    // this position's value quad (not in the cache yet)
    const float4 vcur = *reinterpret_cast<const float4 *>(qkv + qd + kvd + (size_t)g * DH + 4 * dq);
    const int pos = pos_p[0];
    if (pos < 0 || pos >= ctx_len) return;  // the whole block; the step's last kernel reports it
    const int seq = pos + 1, half = rope_dim / 2;
    // Wave w scores the runs w, w + NW, w + 2 NW, ... of CH keys; a wave
    // without keys leaves now (the barrier below waits only for the waves
    // still running).  Wave 0 always has keys.
    const int j0 = wave * CH;
    if (j0 >= seq) return;
    // element i = lane + 64 d: its RoPE pair j and partner element
    int pj_[DPL], pp_[DPL];
    float rc[DPL], rs[DPL];
#pragma unroll
    for (int d = 0; d < DPL; d++) {
        const int i = lane + 64 * d;
        const bool rot = i < 2 * half;
        pj_[d] = rot ? (i < half ? i : i - half) : -1;
        pp_[d] = rot ? (i < half ? i + half : i - half) : i;
        const size_t cb = ((size_t)pos * half + (size_t)(rot ? pj_[d] : 0)) * 2;
        rc[d] = rope_cs[cb];
        rs[d] = rope_cs[cb + 1];
    }
    const float *kbase = k_cache + (size_t)g * DH * ctxp;

    float4 kq[NQD];   // this lane's key, four dimensions per load
    float4 vv[VL];    // value quads of keys kk, kk + KPI, ... of the run
    // A run's cached keys / values, every load unconditional, through
    // buffer resources over this layer's caches (32-bit offsets): key rows
    // at or past pos read row 0 and are unused (the current key's score is
    // formed from registers); value rows at or past pos read past the
    // resource's end, which returns zeros, and the current position's
    // values are added after the run's sums (the last term of its partial
    // sum; the zero products before it leave the sums unchanged).  No
    // select follows a load: one compiles to a branch whose untaken side
    // waits for the load, and the run's loads would no longer be in flight
    // together.
    const __amdgpu_buffer_rsrc_t kres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(kbase), (short)0, (int)(DH * ctxp * sizeof(float)), 0x00020000);
    const __amdgpu_buffer_rsrc_t vres = __builtin_amdgcn_make_buffer_rsrc(
        v_cache, (short)0, (int)(ctxp * kvd * sizeof(float)), 0x00020000);
    const int vlane = (g * DH + 4 * dq) * (int)sizeof(float);
    auto ld4 = [](__amdgpu_buffer_rsrc_t res, int off) {
        typedef unsigned v4u __attribute__((ext_vector_type(4)));
        const v4u t = __builtin_amdgcn_raw_buffer_load_b128(res, off, 0, 0);
        return make_float4(__uint_as_float(t.x), __uint_as_float(t.y), __uint_as_float(t.z), __uint_as_float(t.w));
    };
    auto load_run = [&](int c0) {
        const int r = c0 + lane;
        const int koff = (int)(key_off<DH>(r < pos ? r : 0, 0) * sizeof(float));
#pragma unroll
        for (int i = 0; i < NQD; i++) kq[i] = ld4(kres, koff + 1024 * i);
#pragma unroll
        for (int i = 0; i < VL; i++) {
            const int rj = c0 + i * KPI + kk;
            vv[i] = ld4(vres, rj < pos ? rj * (int)(kvd * sizeof(float)) + vlane : (int)0x80000000);
        }
    };
    load_run(j0);
    __builtin_amdgcn_sched_barrier(0);  // the cache loads go out before any wait below
    // RoPE in registers: the partner element from its lane (both registers
    // when d_head 128), then (a c - b s) for the first of a pair and
    // (a s + b c) for the second, a the first element and b the second.
    auto rope = [&](float (&x)[DPL]) {
        float y[DPL];
#pragma unroll
        for (int d = 0; d < DPL; d++) {
            const int p = pp_[d];
            float xp = lane_val(x[0], p & 63);
            if constexpr (DPL == 2) {
                const float x1 = lane_val(x[1], p & 63);
                xp = p < 64 ? xp : x1;
            }
            const int i = lane + 64 * d;
            if (pj_[d] < 0) {
                y[d] = x[d];
            } else if (i < half) {  // a = x, b = xp
                const float ac = x[d] * rc[d], bs = xp * rs[d];
                y[d] = ac - bs;
            } else {  // a = xp, b = x
                const float as = xp * rs[d], bc = x[d] * rc[d];
                y[d] = as + bc;
            }
        }
#pragma unroll
        for (int d = 0; d < DPL; d++) x[d] = y[d];
    };
    rope(qx);
    rope(kx);
    if (h % qpk == 0 && wave == 0 && !(skip && skip[0])) {  // append this position to the layer's caches
        float *vd = v_cache + (size_t)pos * kvd + (size_t)g * DH;
#pragma unroll
        for (int d = 0; d < DPL; d++) {
            const_cast<float *>(kbase)[key_off<DH>(pos, lane + 64 * d)] = kx[d];
            vd[lane + 64 * d] = vx[d];
        }
    }
    // q to every lane (each lane's dot reads all of it), and, in the wave
    // whose last run holds the current position, that key's score: the
    // reference's sequential dot over the lanes' products q_i k_i.  Both go
    // through the wave's own LDS rows (a wave's LDS accesses complete in
    // order, so no barrier), read back as broadcasts.
    const int c_last = j0 + ((seq - 1 - j0) / (ATT_NW * CH)) * (ATT_NW * CH);  // this wave's last run
    const bool has_pos = pos < c_last + CH;
#pragma unroll
    for (int d = 0; d < DPL; d++) {
        qw[wave][lane + 64 * d] = qx[d];
        pw[wave][lane + 64 * d] = qx[d] * kx[d];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float q[DH];
#pragma unroll
    for (int i = 0; i < DH; i++) q[i] = qw[wave][i];
    float s_pos = 0.0f;
    if (has_pos) {
        float dot = 0.0f;
#pragma unroll
        for (int i = 0; i < DH; i++) dot = dot + pw[wave][i];
        s_pos = dot * scale;
    }
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);  // out[4 dq .. 4 dq + 3]
    float m = -INFINITY, l = 0.0f;
    for (int c0 = j0; c0 < seq; c0 += ATT_NW * CH) {
        const int n = min(CH, seq - c0);
        if (c0 > j0) load_run(c0);
        const bool last = c0 == c_last && has_pos;  // the run holds the current position
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
        if (last && c0 + lane == pos) sc = s_pos;
        const float m_new = fmaxf(m, wave_max(sc));  // finite: the run has a key
        const float corr = rce_exp(m - m_new);           // 0 for the wave's first run
        const float p = lane < n ? rce_exp(sc - m_new) : 0.0f;
        const float lc = l * corr;
        l = lc + wave_sum(p);
        // a[i % NA] sums the keys i KPI + kk: partial sum (i KPI + kk) % 4
        float4 a[NA];
#pragma unroll
        for (int t = 0; t < NA; t++) a[t] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        // every load's p_j first (lane exchanges in flight together), then
        // the sums; p = 0 and zero value rows past the run's keys: whole
        // loads of KPI keys, a uniform test per load (not a break), so the
        // loop unrolls and vv stays in registers
        float pjs[VL];
#pragma unroll
        for (int i = 0; i < VL; i++) pjs[i] = __shfl(p, i * KPI + kk);
#pragma unroll
        for (int i = 0; i < VL; i++) {
            if (i * KPI >= n) continue;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float t = pjs[i] * f4e(vv[i], e);
                f4e(a[i % NA], e) = f4e(a[i % NA], e) + t;
            }
        }
        if (last) {  // the current position's values: key jp's term, last in its partial sum
            const int jp = pos - c0;
            const float pp = rdlane_f32(p, jp);
            if (kk == jp % KPI) {
                float4 &ap = (jp / KPI) % NA == 0 ? a[0] : a[NA - 1];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float t = pp * f4e(vcur, e);
                    f4e(ap, e) = f4e(ap, e) + t;
                }
            }
        }
        // (a0 + a1) + (a2 + a3): with KPI 4 lane group kk holds a_kk; with
        // KPI 2 group kk holds a_kk and a_(kk + 2)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float sv;
            if constexpr (NA == 1) {
                const float x = f4e(a[0], e);
                const float s2 = xor16_sum(x);
                sv = xor32_sum(s2);
            } else {
                const float x0 = f4e(a[0], e), x1 = f4e(a[1], e);
                const float s01 = xor32_sum(x0), s23 = xor32_sum(x1);
                sv = s01 + s23;
            }
            const float oc = f4e(o, e) * corr;
            f4e(o, e) = oc + sv;
        }
        m = m_new;
    }
    float *out = att + (size_t)h * DH;
    if (seq <= CH) {
        // Wave 0 holds every key (the other waves have left): the merge
        // below would weigh it by exp(m - m) = 1 and add it to +0.0, which
        // gives its (o, l) back unchanged (o is never -0.0), so out = o / l
        // directly, without the LDS round trip and the barrier.
        if (kk == 0) {
            const float inv = 1.0f / l;
            float4 r;
#pragma unroll
            for (int e = 0; e < 4; e++) f4e(r, e) = f4e(o, e) * inv;
            *reinterpret_cast<float4 *>(out + 4 * dq) = r;
        }
        return;
    }
    if (kk == 0) *reinterpret_cast<float4 *>(&mo[wave][4 * dq]) = o;
    if (lane == 0) {
        mo[wave][DH] = m;
        mo[wave][DH + 1] = l;
    }
    __syncthreads();
    if (wave != 0) return;
    const int nw = min(ATT_NW, (seq + CH - 1) / CH);  // the waves with keys
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < ATT_NW; w++)
        if (w < nw) M = fmaxf(M, mo[w][DH]);
    float acc[DPL], lacc = 0.0f;
#pragma unroll
    for (int d = 0; d < DPL; d++) acc[d] = 0.0f;
#pragma unroll
    for (int w = 0; w < ATT_NW; w++) {
        if (w >= nw) continue;
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

bool attention_supports(int d_head, int rope_dim, size_t ctx_len, size_t n_kv) {
    const size_t layer_bytes = ((ctx_len + 63) / 64 * 64) * n_kv * (size_t)d_head * sizeof(float);
    return (d_head == 64 || d_head == 128) && rope_dim >= 0 && rope_dim <= d_head && rope_dim % 2 == 0 &&
           layer_bytes < ((size_t)1 << 31);
}

hipError_t launch_attention(const float *qkv, const float *rope_cs, float *k_cache, float *v_cache, const int *pos,
                            int ctx_len, int n_q, int n_kv, int d_head, int rope_dim, float scale, float *att,
                            const int *skip, hipStream_t s) {
    if (n_kv <= 0 || n_q % n_kv || ctx_len <= 0 || !attention_supports(d_head, rope_dim, (size_t)ctx_len, (size_t)n_kv))
        return hipErrorInvalidValue;
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

// moe.hip -- the grouped-expert (MoE) glue kernels of the quantized-matmul
// path: grouping of (token, decision) pairs by expert, gathers, the
// activation between the two expert matrices, and the combine.
//
// Semantics follow rce-qwen36-moe/src/lib.rs L667-710 (moe_ffn_forward: per
// token, per routing decision j, y_j = W2[e] silu(W1[e] x)) and
// rce-op-moe/src/lib.rs L98-110 (moe_combine: out = sum_j w_j * y_j in
// decision order, from +0.0).  The reference loops tokens; here the pairs of
// one expert are stacked into contiguous "slots" so each expert's matrices
// are streamed once for all of its tokens.  The slot order is stable (by
// expert, then token, then decision), so every result is deterministic.
#include "qmm_internal.h"

namespace rce_qmm {
namespace {

constexpr int GT = 256;      // threads of the grouping block
constexpr int GE_MAX = 32;   // experts of the single-scan grouping (LDS counts [GE_MAX][GT])

// Exclusive block scan of one int per thread (GT threads).
__device__ int block_exclusive_scan(int v, int *sh, int &total) {
    const int t = threadIdx.x;
    sh[t] = v;
    __syncthreads();
    for (int off = 1; off < GT; off <<= 1) {
        const int x = t >= off ? sh[t - off] : 0;
        __syncthreads();
        sh[t] += x;
        __syncthreads();
    }
    total = sh[GT - 1];
    const int incl = sh[t];
    __syncthreads();
    return incl - v;
}

// Grouping, done by one block.  Pair p = token * top_k + decision routes
// to expert ids[p].  offs[e] .. offs[e+1]: the slots of expert e;
// slot_of_pair[p]; tok_of_slot[s]; tiles: (expert, first slot, rows <= bm)
// for every bm-row piece of every expert, in expert order; n_tiles[0] =
// their count; status[0] = 1 when an id was out of range (that pair gets no
// slot: slot_of_pair = -1).  Thread t owns the consecutive pairs
// [t * per, (t + 1) * per), so slots in (expert, pair) order are a stable
// counting sort.

// Any expert count: one block scan per expert.
__device__ void group_by_expert_scan(const int32_t *__restrict__ ids, int n_pairs, int top_k, int n_expert, int bm,
                                     int *__restrict__ offs, int *__restrict__ slot_of_pair,
                                     int *__restrict__ tok_of_slot, MoeTile *__restrict__ tiles,
                                     int *__restrict__ n_tiles, int *__restrict__ status, int *sh) {
    const int t = threadIdx.x;
    const int per = (n_pairs + GT - 1) / GT;
    const int p0 = min(n_pairs, t * per), p1 = min(n_pairs, p0 + per);
    int bad = 0;
    for (int p = p0; p < p1; p++) {
        const int e = ids[p];
        if (e < 0 || e >= n_expert) {
            slot_of_pair[p] = -1;
            bad = 1;
        }
    }
    int base = 0, ntile = 0;
    for (int e = 0; e < n_expert; e++) {
        int cnt = 0;
        for (int p = p0; p < p1; p++) cnt += ids[p] == e;
        int total;
        const int before = block_exclusive_scan(cnt, sh, total);
        int s = base + before;
        for (int p = p0; p < p1; p++)
            if (ids[p] == e) {
                slot_of_pair[p] = s;
                tok_of_slot[s] = p / top_k;
                s++;
            }
        if (t == 0) {
            offs[e] = base;
            for (int r = 0; r < total; r += bm) tiles[ntile++] = MoeTile{e, base + r, min(bm, total - r), 0};
        }
        base += total;
    }
    const int any_bad = __syncthreads_or(bad);
    if (t == 0) {
        offs[n_expert] = base;
        n_tiles[0] = ntile;
        status[0] = any_bad;
    }
}

// Up to GE_MAX experts: per-thread counts cnt[e][t] in LDS, one exclusive
// scan of the whole array in (expert, thread) order, which gives every
// (expert, thread) its first slot, then each thread hands out its slots.
__device__ void group_by_expert_counts(const int32_t *__restrict__ ids, int n_pairs, int top_k, int n_expert, int bm,
                                       int *__restrict__ offs, int *__restrict__ slot_of_pair,
                                       int *__restrict__ tok_of_slot, MoeTile *__restrict__ tiles,
                                       int *__restrict__ n_tiles, int *__restrict__ status, int *cnt, int *wsum) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int E = n_expert;
    const int per = (n_pairs + GT - 1) / GT;
    const int p0 = min(n_pairs, t * per), p1 = min(n_pairs, p0 + per);
    for (int e = 0; e < E; e++) cnt[e * GT + t] = 0;
    int bad = 0;
    for (int p = p0; p < p1; p++) {  // own column only: no atomics
        const int e = ids[p];
        if (e < 0 || e >= E) {
            slot_of_pair[p] = -1;
            bad = 1;
        } else {
            cnt[e * GT + t]++;
        }
    }
    __syncthreads();
    // thread t scans the flat entries t*E .. t*E + E - 1 of the (expert, thread) array
    int loc = 0;
    for (int i = 0; i < E; i++) loc += cnt[t * E + i];
    int incl = loc;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(incl, off);
        if (lane >= off) incl += y;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int run = incl - loc, total = 0;
    for (int w = 0; w < GT / 64; w++) {
        if (w < wave) run += wsum[w];
        total += wsum[w];
    }
    for (int i = 0; i < E; i++) {  // flat entries of this thread: read by no other thread here
        const int c = cnt[t * E + i];
        cnt[t * E + i] = run;
        run += c;
    }
    __syncthreads();
    // expert e's first slot is entry (e, 0); tiles in expert order
    if (t < E) {
        const int first = cnt[t * GT], c = (t + 1 < E ? cnt[(t + 1) * GT] : total) - first;
        int tb = 0;
        for (int e = 0; e < t; e++) {
            const int ce = cnt[(e + 1) * GT] - cnt[e * GT];
            tb += (ce + bm - 1) / bm;
        }
        offs[t] = first;
        for (int r = 0; r < c; r += bm) tiles[tb++] = MoeTile{t, first + r, min(bm, c - r), 0};
        if (t == E - 1) {
            offs[E] = total;
            n_tiles[0] = tb;
        }
    }
    __syncthreads();  // column 0 (read above) is thread 0's to advance below
    for (int p = p0; p < p1; p++) {
        const int e = ids[p];
        if (e < 0 || e >= E) continue;
        const int sl = cnt[e * GT + t]++;
        slot_of_pair[p] = sl;
        tok_of_slot[sl] = p / top_k;
    }
    const int any_bad = __syncthreads_or(bad);
    if (t == 0) status[0] = any_bad;
}

// Block 0 groups the pairs; blocks 1.. (when x16 is given) convert the
// f32 activations x[n_x] to binary16 (round to nearest even) for the
// grouped GEMM, independent of the grouping.
__global__ __launch_bounds__(GT) void k_moe_prep(const int32_t *__restrict__ ids, int n_pairs, int top_k, int n_expert,
                                                 int bm, int *__restrict__ offs, int *__restrict__ slot_of_pair,
                                                 int *__restrict__ tok_of_slot, MoeTile *__restrict__ tiles,
                                                 int *__restrict__ n_tiles, int *__restrict__ status,
                                                 const float *__restrict__ x, _Float16 *__restrict__ x16, size_t n_x) {
    __shared__ int cnt[GE_MAX * GT];
    __shared__ int wsum[GT / 64];
    if (blockIdx.x == 0) {
        if (n_expert <= GE_MAX)
            group_by_expert_counts(ids, n_pairs, top_k, n_expert, bm, offs, slot_of_pair, tok_of_slot, tiles, n_tiles,
                                   status, cnt, wsum);
        else
            group_by_expert_scan(ids, n_pairs, top_k, n_expert, bm, offs, slot_of_pair, tok_of_slot, tiles, n_tiles,
                                 status, cnt);
        return;
    }
    const size_t stride = (size_t)(gridDim.x - 1) * GT;
    for (size_t i = (size_t)(blockIdx.x - 1) * GT + threadIdx.x; i < n_x; i += stride) x16[i] = (_Float16)x[i];
}

// xg[s, :] = x[tok_of_slot[s], :]
__global__ void k_gather_rows(const float *__restrict__ x, const int *__restrict__ tok_of_slot, const int *__restrict__ n_slots,
                              size_t d, float *__restrict__ xg) {
    const size_t n = (size_t)n_slots[0] * d;
    for (size_t k = (size_t)blockIdx.x * blockDim.x + threadIdx.x; k < n; k += (size_t)gridDim.x * blockDim.x) {
        const size_t s = k / d, i = k - s * d;
        xg[k] = x[(size_t)tok_of_slot[s] * d + i];
    }
}

__global__ void k_silu_inplace(float *__restrict__ h, const int *__restrict__ n_slots, size_t d) {
    const size_t n = (size_t)n_slots[0] * d;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        h[i] = silu_ref(h[i]);
}

// SwiGLU experts (rce-qwen36-moe/src/lib.rs L667-676 swiglu_expert_serial):
// h = silu(g) * u per slot, in place (f32; the MFMA path forms it in the
// up GEMM's store instead).
__global__ void k_swiglu_slots(float *__restrict__ g, const float *__restrict__ u, const int *__restrict__ n_slots,
                               size_t d) {
    const size_t n = (size_t)n_slots[0] * d;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        g[i] = silu_ref(g[i]) * u[i];
}

// moe_combine (rce-op-moe/src/lib.rs L98-110): out[t, :] = sum_j w[t, j] * y[slot(t, j), :],
// j in decision order, from +0.0; a pair without a slot contributes nothing.
// Block (t, c): token t, columns 1024 c .. 1024 c + 1023 (and every
// gridDim.y-th such range after), four per thread (d a multiple of 4), so
// a thread's loads of y are one float4 per decision, all in flight at once.
__global__ __launch_bounds__(256) void k_moe_combine4(const float *__restrict__ y, const int *__restrict__ slot_of_pair,
                                                      const float *__restrict__ gate_w, int top_k, size_t d,
                                                      float *__restrict__ out) {
    const size_t t = blockIdx.x, d4 = d / 4;
    const float4 *y4 = reinterpret_cast<const float4 *>(y);
    float4 *o4 = reinterpret_cast<float4 *>(out) + t * d4;
    for (size_t i = (size_t)blockIdx.y * 256 + threadIdx.x; i < d4; i += (size_t)gridDim.y * 256) {
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int j = 0; j < top_k; j++) {
            const int s = slot_of_pair[t * top_k + j];
            if (s < 0) continue;
            const float w = gate_w[t * top_k + j];
            const float4 v = y4[(size_t)s * d4 + i];
            const float px = w * v.x, py = w * v.y, pz = w * v.z, pw = w * v.w;
            acc.x += px;
            acc.y += py;
            acc.z += pz;
            acc.w += pw;
        }
        o4[i] = acc;
    }
}

__global__ void k_moe_combine(const float *__restrict__ y, const int *__restrict__ slot_of_pair,
                              const float *__restrict__ gate_w, int top_k, size_t t_rows, size_t d,
                              float *__restrict__ out) {
    for (size_t k = (size_t)blockIdx.x * blockDim.x + threadIdx.x; k < t_rows * d; k += (size_t)gridDim.x * blockDim.x) {
        const size_t t = k / d, i = k - t * d;
        float acc = 0.0f;
        for (int j = 0; j < top_k; j++) {
            const int s = slot_of_pair[(size_t)t * top_k + j];
            if (s < 0) continue;
            const float prod = gate_w[(size_t)t * top_k + j] * y[(size_t)s * d + i];
            acc += prod;
        }
        out[k] = acc;
    }
}

unsigned grid_1d(size_t n, unsigned bs) {
    size_t g = (n + bs - 1) / bs;
    return (unsigned)(g < 8192 ? (g ? g : 1) : 8192);
}

}  // namespace

hipError_t launch_moe_group(const int32_t *ids, size_t n_pairs, int top_k, int n_expert, int bm, int *offs,
                            int *slot_of_pair, int *tok_of_slot, MoeTile *tiles, int *n_tiles, int *status,
                            const float *x, void *x16, size_t n_x, hipStream_t s) {
    const unsigned conv = x16 && n_x ? grid_1d(n_x, GT) : 0;
    const unsigned blocks = 1 + (conv < 1024 ? conv : 1024);
    hipLaunchKernelGGL(k_moe_prep, dim3(blocks), dim3(GT), 0, s, ids, (int)n_pairs, top_k, n_expert, bm, offs,
                       slot_of_pair, tok_of_slot, tiles, n_tiles, status, x, static_cast<_Float16 *>(x16), n_x);
    return hipGetLastError();
}

hipError_t launch_gather_rows(const float *x, const int *tok_of_slot, const int *n_slots_dev, size_t max_slots,
                              size_t d, float *xg, hipStream_t s) {
    if (max_slots == 0) return hipSuccess;
    hipLaunchKernelGGL(k_gather_rows, dim3(grid_1d(max_slots * d, 256)), dim3(256), 0, s, x, tok_of_slot, n_slots_dev, d,
                       xg);
    return hipGetLastError();
}

hipError_t launch_silu_inplace(float *h, const int *n_slots_dev, size_t max_slots, size_t d, hipStream_t s) {
    hipLaunchKernelGGL(k_silu_inplace, dim3(grid_1d(max_slots * d, 256)), dim3(256), 0, s, h, n_slots_dev, d);
    return hipGetLastError();
}

hipError_t launch_swiglu_slots(float *g, const float *u, const int *n_slots_dev, size_t max_slots, size_t d,
                               hipStream_t s) {
    hipLaunchKernelGGL(k_swiglu_slots, dim3(grid_1d(max_slots * d, 256)), dim3(256), 0, s, g, u, n_slots_dev, d);
    return hipGetLastError();
}

hipError_t launch_moe_combine(const float *y, const int *slot_of_pair, const float *gate_w, size_t t_rows, int top_k,
                              size_t d, float *out, hipStream_t s) {
    if (t_rows == 0) return hipSuccess;
    if (d % 4 == 0 && t_rows <= 0xFFFFFFFFu / 256) {  // grid.x * 256 threads within 32 bits
        const size_t cy = d >= 4 ? (d / 4 + 255) / 256 : 1;
        hipLaunchKernelGGL(k_moe_combine4, dim3((unsigned)t_rows, (unsigned)(cy < 65535 ? cy : 65535)), dim3(256), 0, s, y,
                           slot_of_pair, gate_w, top_k, d, out);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_moe_combine, dim3(grid_1d(t_rows * d, 256)), dim3(256), 0, s, y, slot_of_pair, gate_w, top_k,
                       t_rows, d, out);
    return hipGetLastError();
}

}  // namespace rce_qmm

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

constexpr int GT = 256;  // threads of the grouping block

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

// One block.  Pair p = token * top_k + decision routes to expert ids[p].
// offs[e] .. offs[e+1]: the slots of expert e; slot_of_pair[p]; tok_of_slot[s];
// tiles: (expert, first slot, rows <= bm) for every bm-row piece of every
// expert, in expert order; n_tiles[0] = their count; status[0] = 1 when an
// id was out of range (that pair gets no slot: slot_of_pair = -1).
__global__ __launch_bounds__(GT) void k_moe_group(const int32_t *__restrict__ ids, int n_pairs, int top_k, int n_expert,
                                                  int bm, int *__restrict__ offs, int *__restrict__ slot_of_pair,
                                                  int *__restrict__ tok_of_slot, MoeTile *__restrict__ tiles,
                                                  int *__restrict__ n_tiles, int *__restrict__ status) {
    __shared__ int sh[GT];
    const int t = threadIdx.x;
    const int per = (n_pairs + GT - 1) / GT;  // consecutive pairs per thread
    const int p0 = t * per, p1 = min(n_pairs, p0 + per);
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
    // any thread that saw a bad id reports it
    const int any_bad = __syncthreads_or(bad);
    if (t == 0) {
        offs[n_expert] = base;
        n_tiles[0] = ntile;
        status[0] = any_bad;
    }
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

__global__ void k_silu_f16(const float *__restrict__ h, _Float16 *__restrict__ o, const int *__restrict__ n_slots,
                           size_t d) {
    const size_t n = (size_t)n_slots[0] * d;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        o[i] = (_Float16)silu_ref(h[i]);
}

// SwiGLU experts (rce-qwen36-moe/src/lib.rs L667-676 swiglu_expert_serial):
// h = silu(g) * u per slot, in place (f32) or into binary16 for the MFMA GEMM.
__global__ void k_swiglu_slots(float *__restrict__ g, const float *__restrict__ u, const int *__restrict__ n_slots,
                               size_t d) {
    const size_t n = (size_t)n_slots[0] * d;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        g[i] = silu_ref(g[i]) * u[i];
}

__global__ void k_swiglu_slots_f16(const float *__restrict__ g, const float *__restrict__ u, _Float16 *__restrict__ o,
                                   const int *__restrict__ n_slots, size_t d) {
    const size_t n = (size_t)n_slots[0] * d;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        o[i] = (_Float16)(silu_ref(g[i]) * u[i]);
}

// moe_combine (rce-op-moe/src/lib.rs L98-110): out[t, :] = sum_j w[t, j] * y[slot(t, j), :],
// j in decision order, from +0.0; a pair without a slot contributes nothing.
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
                            hipStream_t s) {
    hipLaunchKernelGGL(k_moe_group, dim3(1), dim3(GT), 0, s, ids, (int)n_pairs, top_k, n_expert, bm, offs,
                       slot_of_pair, tok_of_slot, tiles, n_tiles, status);
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

hipError_t launch_silu_f16(const float *h, void *o, const int *n_slots_dev, size_t max_slots, size_t d,
                           hipStream_t s) {
    hipLaunchKernelGGL(k_silu_f16, dim3(grid_1d(max_slots * d, 256)), dim3(256), 0, s, h, static_cast<_Float16 *>(o),
                       n_slots_dev, d);
    return hipGetLastError();
}

hipError_t launch_swiglu_slots(float *g, const float *u, const int *n_slots_dev, size_t max_slots, size_t d,
                               hipStream_t s) {
    hipLaunchKernelGGL(k_swiglu_slots, dim3(grid_1d(max_slots * d, 256)), dim3(256), 0, s, g, u, n_slots_dev, d);
    return hipGetLastError();
}

hipError_t launch_swiglu_slots_f16(const float *g, const float *u, void *o, const int *n_slots_dev, size_t max_slots,
                                   size_t d, hipStream_t s) {
    hipLaunchKernelGGL(k_swiglu_slots_f16, dim3(grid_1d(max_slots * d, 256)), dim3(256), 0, s, g, u,
                       static_cast<_Float16 *>(o), n_slots_dev, d);
    return hipGetLastError();
}

hipError_t launch_moe_combine(const float *y, const int *slot_of_pair, const float *gate_w, size_t t_rows, int top_k,
                              size_t d, float *out, hipStream_t s) {
    if (t_rows == 0) return hipSuccess;
    hipLaunchKernelGGL(k_moe_combine, dim3(grid_1d(t_rows * d, 256)), dim3(256), 0, s, y, slot_of_pair, gate_w, top_k,
                       t_rows, d, out);
    return hipGetLastError();
}

}  // namespace rce_qmm

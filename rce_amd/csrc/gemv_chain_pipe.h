// gemv_chain_pipe.h -- the chain wave's side of the stage pipeline of the
// row-chain GEMVs (gemv_chain.hip: F32 / F16 / BF16, I2_S; gemv_q6_k.hip:
// Q6_K EXACT).  In those formats the reference sums a row as one chain of
// dependent f32 adds, so one lane holds each chain and helper waves form
// the addends: per stage of SV addends they write them to LDS slot s % 2 as
// float4 (addends 4q .. 4q + 3 of a chain at prod[(slot * SV / 4 + q) * LN]),
// and meet the chain wave at one barrier per stage.
#pragma once

#include <hip/hip_runtime.h>

namespace rce_qmm {

// s_tot barriers; after barrier s the stage s addends are in slot s % 2
// (prod already at the lane's chain).  Half stages rotate through two
// register sets: the reads of one half are issued before the adds of the
// half before it, so the LDS latency hides behind 4 * (SV / 8) adds, and
// the chain adds every stage below ns in order.
template <int SV, int LN>
__device__ __forceinline__ float run_chain(const float4 *prod, int ns, int s_tot) {
    constexpr int HQ = SV / 8;  // float4 per half stage
    static_assert(HQ * 8 == SV, "half stages of whole float4");
    float4 r1[HQ], r2[HQ];
    float acc = 0.0f;
    auto rd = [&](int s, int half, float4 *v) {
        const float4 *p = prod + ((size_t)(s & 1) * (SV / 4) + half * HQ) * LN;
#pragma unroll
        for (int q = 0; q < HQ; q++) v[q] = p[q * LN];
    };
    auto add = [&](int s, const float4 *v) {
        if (s >= ns) return;
#pragma unroll
        for (int q = 0; q < HQ; q++) {
            acc = acc + v[q].x;
            acc = acc + v[q].y;
            acc = acc + v[q].z;
            acc = acc + v[q].w;
        }
    };
    __syncthreads();
    rd(0, 0, r1);
    rd(0, 1, r2);
    add(0, r1);
    for (int s = 1; s < s_tot; s++) {
        __syncthreads();  // stage s written; stage s - 1's slot free for stage s + 1
        rd(s, 0, r1);
        add(s - 1, r2);
        rd(s, 1, r2);
        add(s, r1);
    }
    add(s_tot - 1, r2);
    return acc;
}

// Copy a token's k activations to LDS act[0 .. kp), zeros past k, with all
// NT threads: the loads of a round first, then the stores; stores past kp
// go to act[kp] (a dump slot the caller allocates), so no store sits in a
// branch (a branch's skipped wait would leave the loads pending, as far as
// the compiler can tell, and every later reuse of their registers would
// wait for all loads in flight).  MAP(i) is the LDS index of element i < k.
template <int NT, int U, class Map>
__device__ __forceinline__ void stage_act(const float *__restrict__ a, size_t k, size_t kp, float *act, Map map) {
    const int tid = threadIdx.x;
    for (size_t i0 = 0; i0 < kp; i0 += (size_t)NT * U) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const size_t i = i0 + (size_t)u * NT + tid;
            v[u] = a[i < k ? i : k - 1];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const size_t i = i0 + (size_t)u * NT + tid;
            act[i < k ? map(i) : (i < kp ? i : kp)] = i < k ? v[u] : 0.0f;
        }
    }
}

}  // namespace rce_qmm

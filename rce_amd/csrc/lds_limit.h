// lds_limit.h -- raising a kernel's dynamic LDS limit above HIP's default
// 64 KB (gfx950 has 160 KB per CU).  The limit is an attribute of the
// function on a device, so it is set once per (function, device); the
// record is shared by every thread of the process.
#pragma once

#include <hip/hip_runtime.h>

#include <mutex>
#include <set>
#include <utility>

namespace rce_qmm {

inline hipError_t ensure_lds_limit(const void *fn, int bytes) {
    static std::mutex mu;
    static std::set<std::pair<const void *, int>> done;  // (function, device)
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(mu);
    if (done.count({fn, dev})) return hipSuccess;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess) done.insert({fn, dev});
    return e;
}

// Raise the limit, on the current device, for every kernel of the row-chain
// GEMVs that can need more than 64 KB (gemv_chain.hip, gemv_q6_k.hip).
// Called when a context binds its device, so that no first launch sets an
// attribute while a stream is being captured into a graph.
hipError_t chain_prepare_lds();
hipError_t q6_prepare_lds();
// The same for every instantiation of the prefill / grouped GEMM (gemm_f16.hip).
hipError_t gemm_prepare_lds();

}  // namespace rce_qmm

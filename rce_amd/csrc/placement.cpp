// placement.cpp -- the "hip:op-qmm" priced backend's cost side for
// rce-placement-adapter (src/lib.rs L118-160, L130-283): the adapter's qmm
// dtype IDs, the decline rule (cost = +inf for a weight the GPU does not
// compute, so pick_priced routes it to CpuQmm), the (flops, bytes) features
// of qmm_1d_flops_bytes (L141-145) and the library's analytical prior for
// the ("qmm", "hip:op-qmm") cost cell.  Dispatch itself is rce_qmm_mm_1d.
#include "abi_internal.h"

#include <limits>

using namespace rce_qmm;
using namespace rce_qmm_abi;

extern "C" {

// QMM_DTYPE_* (rce-placement-adapter/src/lib.rs L80-90) -> GGUF tag; 0 for
// QMM_DTYPE_UNKNOWN and unassigned ids.
uint32_t rce_qmm_dtype_for_qmm_id(size_t qmm_dtype_id) {
    static const uint32_t tag[] = {0, 8, 12, 13, 14, 2, 6, 3, 41, 42, 11};
    return qmm_dtype_id < sizeof(tag) / sizeof(tag[0]) ? tag[qmm_dtype_id] : 0;
}

// Analytical prior (basis est) for the ("qmm", "hip:op-qmm") cell, on the
// scale of the reference's own priors (cpu:op-qmm a = 10 pJ/FLOP, b = 0.05
// pJ/B, c = 5e5 pJ; default_qmm_cost_table L163-182).  Derived from measured
// times: the headline GEMV (Q4_0 11008x4096) runs about 100x faster on one
// MI355X than the reference-order CPU path on 16 host cores, at about 14x the
// board power, so a = 10 / 9; a host-entry call (copy in, launch, copy out,
// sync: 28.6 us for a 64x64 weight) costs about 3x the CPU path's fixed
// per-call time (9.7 us) at that power ratio, so c = 5e5 * 42; the per-byte
// term stays the reference's 0.05.
void rce_qmm_hip_cost_prior(double *a_pj_per_flop, double *b_pj_per_byte, double *c_pj_overhead) {
    if (a_pj_per_flop) *a_pj_per_flop = 10.0 / 9.0;
    if (b_pj_per_byte) *b_pj_per_byte = 0.05;
    if (c_pj_overhead) *c_pj_overhead = 5.0e5 * 42.0;
}

// HipQmm::cost for op "qmm": a_shape = [k], w_shape = [n_rows, n_cols,
// weight_bytes, dtype_id] (PlacementQmmAdapter::qmm_1d L425-438).  +inf when
// the shapes are short, the dtype id has no GGUF tag here, or the GPU has no
// kernel for (tag, n_cols); else a*flops + b*bytes + c with flops = 2 n k and
// bytes = weight_bytes + 4 k + 4 n.
rce_qmm_status rce_qmm_hip_cost(const size_t *a_shape, size_t a_len, const size_t *w_shape, size_t w_len,
                                double a_pj_per_flop, double b_pj_per_byte, double c_pj_overhead,
                                double *picojoules) {
    if (!picojoules || (a_len && !a_shape) || (w_len && !w_shape)) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    const double inf = std::numeric_limits<double>::infinity();
    *picojoules = inf;
    if (a_len < 1 || w_len < 2) return RCE_QMM_OK;
    const uint32_t tag = rce_qmm_dtype_for_qmm_id(w_len > 3 ? w_shape[3] : 0);
    if (tag == 0 || !gpu_supports(tag, w_shape[1], RCE_QMM_MODE_EXACT)) return RCE_QMM_OK;
    const double k = (double)a_shape[0], n = (double)w_shape[0];
    const double wb = w_len > 2 ? (double)w_shape[2] : 0.0;
    const double flops = 2.0 * n * k, bytes = wb + 4.0 * k + 4.0 * n;
    *picojoules = a_pj_per_flop * flops + b_pj_per_byte * bytes + c_pj_overhead;
    return RCE_QMM_OK;
}

}  // extern "C"

// gemm_epilogue.h -- the SiLU of the matrix-core GEMMs' grouped-expert
// epilogues (mode F16_MFMA), whose result is rounded to binary16.
#pragma once

#include <hip/hip_runtime.h>

namespace rce_qmm {

// silu(x) = x * sigmoid(x) with the hardware's 2^x (v_exp_f32) and
// reciprocal (v_rcp_f32): relative error about 1e-6, far below the binary16
// rounding (2^-11) that follows, and branch-free.  The bit-exact modes keep
// silu_ref (the reference's x / (1 + exp(-x)) with rce_exp); evaluating that
// in both branches of a wave cost about 60 VALU instructions per output and
// a quarter of the expert GEMM's epilogue.  Large negative x gives -0 (the
// reference's value rounds to it), +-inf and NaN give NaN as x / (1 + e^-x)
// does at -inf and NaN; +inf gives +inf.
__device__ __forceinline__ float silu_mfma(float x) {
    const float e = __builtin_amdgcn_exp2f(-x * 1.44269504088896341f);
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

}  // namespace rce_qmm

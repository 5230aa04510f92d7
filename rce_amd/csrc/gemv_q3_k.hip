// gemv_q3_k.hip -- the Q3_K decode kernels (EXACT and Q8).
#include "qmm_gemv_kernels.h"

namespace rce_qmm {
hipError_t launch_gemv_q3_k(const DevWeight &w, const GemvGeom &g, const float *a, size_t t_rows, float *out, int mode,
                            hipStream_t s) {
    if (mode == 0) return launch_as_tb<Q3_KExact, false, 4>(w, g, a, t_rows, out, s);
    return launch_as_tb<Q3_KQ8, true, 8>(w, g, a, t_rows, out, s);
}
hipError_t launch_gemv_fx_q3_k(const FxLaunch &f, const GemvGeom &g, const float *a, int mode, hipStream_t s) {
    if (mode == 0) return launch_as_fx_nt<Q3_KExact<1>, false>(f, g, a, s);
    return launch_as_fx_nt<Q3_KQ8<1>, true>(f, g, a, s);
}
}  // namespace rce_qmm

// zlm_gemv_timeline.hip -- timeline instances of two GEMVs (the same template
// instantiations as the library's kernels, plus the per-wave s_memrealtime
// points of Timeline<true>), loaded only by gemv_timeline.cpp to show where a
// launch's time goes: the configs[1] gate/up GEMV (zlm_gemv_q8_0_r1_s4) and
// the decode step's RMSNorm + gate/up + SiLU (zlm_gemv_q4_0_normpair_s2_pfqw16).
#include "gemv_impl.h"

extern "C" __global__ void __launch_bounds__(256)
    zlm_tl_q8_0_r1_s4(const uint8_t* __restrict__ w, const uint16_t* __restrict__ dsc, const float* __restrict__ x,
                      float* __restrict__ y, uint32_t rows, uint32_t nb, uint64_t* tl) {
    GemvArgs a = {w, dsc, w, dsc, x, x, y, y, rows, nb, 0.0f, 0u};
    gemv<Q8_0, 4096, 4, 1, 4, true, true, PRO_PLAIN, EPI_PLAIN, false, false, false, true>(a, tl);
}

extern "C" __global__ void __launch_bounds__(1024) zlm_tl_q4_0_normpair_s2_pfqw16(GemvArgs a, uint64_t* tl) {
    gemv<Q4_0, 4096, 16, 2, 2, true, true, PRO_NORM, EPI_PAIR, true, false, true, true>(a, tl);
}

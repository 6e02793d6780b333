// zlm_gemv_q4_0.hip -- the q4_0 GEMV entry points (plain and fused forms),
// built as their own gfx950 code object so the instance files compile in
// parallel.
#include "gemv_impl.h"

ZLM_GEMV_Q4(q4_0, Q4_0)
ZLM_GEMVX_Q4(q4_0, Q4_0)
ZLM_GEMVX_FORMS(q4_0, Q4_0, 16384, 6, true, s6)

// Prefetching forms for the decode-step shapes (measured on gfx950 against
// the forms above: gate_up 12288 x 4096 15.3 -> 13.1 us with 8-wave
// workgroups; down 4096 x 12288 12.9 -> 10.4 us with a 12288-float x, so two
// workgroups fit a CU's LDS).
ZLM_GEMVX_PF(zlm_gemv_q4_0_pair_s2_pf, Q4_0, 4096, 8, 2, 2, PRO_PLAIN, EPI_PAIR, false)
ZLM_GEMVX_PF(zlm_gemv_q4_0_normpair_s2_pf, Q4_0, 4096, 8, 2, 2, PRO_NORM, EPI_PAIR, false)
ZLM_GEMVX_PF(zlm_gemv_q4_0_resid_s6_pf, Q4_0, 12288, 4, 1, 6, PRO_PLAIN, EPI_RESID, true)

ZLM_GEMV_MULTI_Q4(q4_0, Q4_0)

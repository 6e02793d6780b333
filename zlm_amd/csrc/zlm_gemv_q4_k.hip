// zlm_gemv_q4_k.hip -- the q4_k GEMV entry points (plain and fused forms),
// built as their own gfx950 code object so the instance files compile in
// parallel.
#include "gemv_impl.h"

ZLM_GEMV_Q4_COMMON(q4_k, Q4_K)
ZLM_GEMVX_Q4(q4_k, Q4_K)

// Prefetching plain instance for 14336 < k <= 16384 (measured on gfx950 at
// 3840 x 15360: 19.2 -> 16.6 us with 8-wave workgroups at 8 waves per CU).
ZLM_GEMVX_PF(zlm_gemv_q4_k_r1_s8_pf, Q4_K, 16384, 8, 1, 8, PRO_PLAIN, EPI_PLAIN, true)

ZLM_GEMV_MULTI_Q4(q4_k, Q4_K)

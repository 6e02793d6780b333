// zlm_gemv_q6_k.hip -- the q6_k GEMV entry points (plain and fused forms),
// built as their own gfx950 code object so the instance files compile in
// parallel.
#include "gemv_impl.h"

ZLM_GEMV_Q4_COMMON(q6_k, Q6_K)
ZLM_GEMVX_Q4(q6_k, Q6_K)

// Prefetching plain instance for k <= 4096 (measured on gfx950 at 15360 x
// 3840: 16.3 -> 12.9 us with 8-wave workgroups at 8 waves per CU).
ZLM_GEMVX_PF(zlm_gemv_q6_k_r1_s2_pf, Q6_K, 4096, 8, 1, 2, PRO_PLAIN, EPI_PLAIN, false)

// Split-K form for 7 < chunks/64 <= 8 (the C3 down projection 3840 x 15360):
// 8-wave workgroups, one per CU, two rows per tile; measured on gfx950 19.5 ->
// 14.8 us against the 4-wave exact-steps instance.
ZLM_GEMV_SK(zlm_gemv_q6_k_r1_s8_sk2, Q6_K, 8, 2, 1, EPI_PLAIN, false, 2, false)

ZLM_GEMV_MULTI_Q4(q6_k, Q6_K)

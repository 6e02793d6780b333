// zlm_gemv_q4_k.hip -- the q4_k GEMV entry points (plain and fused forms),
// built as their own gfx950 code object so the instance files compile in
// parallel.
#include "gemv_impl.h"

ZLM_GEMV_Q4_COMMON(q4_k, Q4_K)
ZLM_GEMVX_Q4(q4_k, Q4_K)

// Prefetching plain instance for 14336 < k <= 16384 (measured on gfx950 at
// 3840 x 15360: 19.2 -> 16.6 us with 8-wave workgroups at 8 waves per CU).
ZLM_GEMVX_PF(zlm_gemv_q4_k_r1_s8_pf, Q4_K, 16384, 8, 1, 8, PRO_PLAIN, EPI_PLAIN, true)

// Split-K form for 7 < chunks/64 <= 8 (the C3 down projection 3840 x 15360):
// 8-wave workgroups, one per CU, two rows per tile; measured on gfx950 16.6 ->
// 13.0 us against the prefetching instance above.
ZLM_GEMV_SK(zlm_gemv_q4_k_r1_s8_sk2, Q4_K, 8, 2, 1, EPI_PLAIN, false, 2, false)

ZLM_GEMV_MULTI_Q4(q4_k, Q4_K)

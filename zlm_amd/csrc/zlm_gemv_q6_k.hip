// zlm_gemv_q6_k.hip -- the q6_k GEMV entry points (plain and fused forms),
// built as their own gfx950 code object so the instance files compile in
// parallel.
#include "gemv_impl.h"

ZLM_GEMV_Q4_COMMON(q6_k, Q6_K)
ZLM_GEMVX_Q4(q6_k, Q6_K)

// Prefetching plain instance for k <= 4096 (measured on gfx950 at 15360 x
// 3840: 16.3 -> 12.9 us with 8-wave workgroups at 8 waves per CU).
ZLM_GEMVX_PF(zlm_gemv_q6_k_r1_s2_pf, Q6_K, 4096, 8, 1, 2, PRO_PLAIN, EPI_PLAIN, false)

// The lm_head (from 65536 rows, k <= 4096): x as int8 planes (v_dot4 on the
// 6-bit quants), prefetching 8-wave workgroups at 16 waves per CU; measured on
// gfx950 at 262144 x 3840: 190.7 -> 156.5 us against the 4-wave exact-steps
// instance at 8 workgroups per CU.  At 15360 rows the int8 planes do not pay
// (12.9 vs 13.5 us), so the _pf instance above stays fp32.
ZLM_GEMVX_PFQ(zlm_gemv_q6_k_r1_s2_tallq, Q6_K, 4096, 8, 1, 2, PRO_PLAIN, EPI_PLAIN, false)

// Split-K form for 7 < chunks/64 <= 8 (the C3 down projection 3840 x 15360):
// 8-wave workgroups, one per CU, two rows per tile; measured on gfx950 19.5 ->
// 14.8 us against the 4-wave exact-steps instance.
ZLM_GEMV_SK(zlm_gemv_q6_k_r1_s8_sk2, Q6_K, 8, 2, 1, EPI_PLAIN, false, 2, false)

ZLM_GEMV_MULTI_Q4(q6_k, Q6_K)

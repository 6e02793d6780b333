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
// 8-wave workgroups, one per CU, four rows per tile, x as int8 planes in
// registers; measured on gfx950 16.7 -> 12.2 us against the prefetching
// instance above (13.0 us with fp32 x and two rows per tile), 10.7 us on the
// qs + record layout, 10.4 us with the parked reduction (one barrier per 16
// tiles instead of one per tile).
ZLM_GEMV_SKP(zlm_gemv_q4_k_r1_s8_sk4, Q4_K, 8, 4, 1, EPI_PLAIN, true, 2, false, 16)
// The same for the other long rows (k 8193-20480, e.g. 11008, 14336, 17408).
ZLM_GEMV_SKP(zlm_gemv_q4_k_r1_s5_sk4, Q4_K, 5, 4, 1, EPI_PLAIN, true, 2, false, 16)
ZLM_GEMV_SKP(zlm_gemv_q4_k_r1_s6_sk4, Q4_K, 6, 4, 1, EPI_PLAIN, true, 2, false, 16)
ZLM_GEMV_SKP(zlm_gemv_q4_k_r1_s7_sk4, Q4_K, 7, 4, 1, EPI_PLAIN, true, 2, false, 16)
ZLM_GEMV_SKP(zlm_gemv_q4_k_r1_s9_sk4, Q4_K, 9, 4, 1, EPI_PLAIN, true, 2, false, 16)
ZLM_GEMV_SKP(zlm_gemv_q4_k_r1_s10_sk4, Q4_K, 10, 4, 1, EPI_PLAIN, true, 2, false, 16)
ZLM_GEMV_SKP(zlm_gemv_q4_k_r1_s3_sk4, Q4_K, 3, 4, 1, EPI_PLAIN, true, 2, false, 16)
ZLM_GEMV_SKP(zlm_gemv_q4_k_r1_s4_sk4, Q4_K, 4, 4, 1, EPI_PLAIN, true, 2, false, 16)

// k <= 4096 (the C3 gate/up 15360 x 3840): x as int8 planes, prefetching
// 16-wave workgroups, one per CU (the x planes are built once per 16 waves);
// 11.6 -> 10.9 us (8-wave groups on the raw blocks) -> 9.1 us on the qs +
// record layout, against the 4-wave exact-steps instance at 4 workgroups per CU.
ZLM_GEMVX_PFQ(zlm_gemv_q4_k_r1_s2_pfqw16, Q4_K, 4096, 16, 1, 2, PRO_PLAIN, EPI_PLAIN, false)

ZLM_GEMV_MULTI_Q4(q4_k, Q4_K)

// matMul at m = 2 (both tokens in one pass over the weights)
ZLM_GEMV_TOK2(q4_k, Q4_K, 2)
ZLM_GEMVTR(zlm_gemv_q4_k_tok2_g4_r2, Q4_K, 4096, 4, 2, 2)
ZLM_GEMVTR(zlm_gemv_q4_k_tok2_g4_r4, Q4_K, 4096, 4, 4, 2)
ZLM_GEMVTR(zlm_gemv_q4_k_tok2_g8_r2, Q4_K, 8192, 8, 2, 2)

// matMul at m = 3, 4 (int path, the weights read once for all tokens)
ZLM_GEMV_Q8TOK(q4_k, Q4_K, 2)
ZLM_GEMV_Q8TOK8(q4_k, Q4_K, 2)
ZLM_GEMV_Q8TOK16(q4_k, Q4_K, 2)
ZLM_GEMV_Q8TOK_R2(q4_k, Q4_K, 2)

// Rows of 4097-8192 elements: the generic two-step loop over an 8192-element
// x tile, where the host takes it (measured faster than the exact-steps forms)
ZLM_GEMV_G8K(q4_k, Q4_K)
// The lm_heads at 3-4 chunk steps (k 4097-8192, from 65536 rows): prefetching
// 8-wave workgroups at 16 waves per CU with x as int8 planes, two-row wave
// tiles at 3 steps.  Measured on gfx950 against the exact-steps instances
// (alternating runs, weights rotated past the Infinity Cache): 152064 x 5120
// 123 -> 106 us, 128256 x 8192 141 -> 124 us.  At 2 steps the one-row form
// matched the 16-wave pfqw16 instance (151936 x 4096: 81 us either way).
ZLM_GEMVX_PFQ(zlm_gemv_q4_k_r2_s3_tallq, Q4_K, 8192, 8, 2, 3, PRO_PLAIN, EPI_PLAIN, false)
ZLM_GEMVX_PFQ(zlm_gemv_q4_k_r1_s4_tallq1, Q4_K, 8192, 8, 1, 4, PRO_PLAIN, EPI_PLAIN, false)
// The RMSNorm-fused lm_heads at 3-4 chunk steps (from 65536 rows).  Measured
// on gfx950 (graph replays, weights rotated past the Infinity Cache): 152064
// x 5120 119 -> 98 us, 128256 x 8192 133 -> 114 us.
ZLM_GEMVX_PFQ(zlm_gemv_q4_k_norm_s3_tallq, Q4_K, 8192, 8, 2, 3, PRO_NORM, EPI_PLAIN, false)
ZLM_GEMVX_PFQ(zlm_gemv_q4_k_norm_s4_tallq1, Q4_K, 8192, 8, 1, 4, PRO_NORM, EPI_PLAIN, false)

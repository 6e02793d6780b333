// zlm_gemv_q6_k.hip -- the q6_k GEMV entry points (plain and fused forms),
// built as their own gfx950 code object so the instance files compile in
// parallel.
#include "gemv_impl.h"

ZLM_GEMV_Q4_COMMON(q6_k, Q6_K)
ZLM_GEMVX_Q4(q6_k, Q6_K)

// k <= 4096 below 65536 rows (the C3 gate/up 15360 x 3840): x as int8 planes
// (v_dot4 on the 6-bit quants), prefetching 16-wave workgroups, one per CU (the
// planes are built once per 16 waves).  Measured on gfx950 at 15360 x 3840:
// 16.3 -> 12.9 us with the fp32-x 8-wave prefetching instance on the 208-byte
// blocks, 11.8 us here on the ql + record layout.
ZLM_GEMVX_PFQ(zlm_gemv_q6_k_r1_s2_pfqw16, Q6_K, 4096, 16, 1, 2, PRO_PLAIN, EPI_PLAIN, false)

// The lm_head (from 65536 rows, k <= 4096): x as int8 planes, prefetching
// 8-wave workgroups at 16 waves per CU, two rows per wave tile; measured on
// gfx950 at 262144 x 3840: 190.7 -> 156.5 us against the 4-wave exact-steps
// instance, 147.7 us on the ql + record layout, 140.8 us with two-row tiles.
// The same at 3 steps (k 4097-6144; 235 VGPRs, two waves per SIMD, so one
// resident 8-wave workgroup per CU): 152064 x 5120 161 -> 134 us against the
// generic two-step instance, 65536 x 5120 81 -> 71 us; at 4 steps the
// one-row form measured slower than the exact-steps instance (190 against
// 183 us at 152064 x 8192) and is not built.
ZLM_GEMVX_PFQ(zlm_gemv_q6_k_r2_s2_tallq, Q6_K, 4096, 8, 2, 2, PRO_PLAIN, EPI_PLAIN, false)
ZLM_GEMVX_PFQ(zlm_gemv_q6_k_r2_s3_tallq, Q6_K, 8192, 8, 2, 3, PRO_PLAIN, EPI_PLAIN, false)

// Split-K form for 7 < chunks/64 <= 8 (the C3 down projection 3840 x 15360):
// 8-wave workgroups, one per CU, two rows per tile; measured on gfx950 19.5 ->
// 14.8 us against the 4-wave exact-steps instance, 13.1 us on the ql + record
// layout, 12.5 us with the parked reduction (one barrier per 16 tiles).  The
// q8_0 / q4_0 split-K downs measured slower parked (10.6 -> 11.4, 9.1 -> 9.5
// us) and keep one barrier per tile.
ZLM_GEMV_SKP(zlm_gemv_q6_k_r1_s8_sk2, Q6_K, 8, 2, 1, EPI_PLAIN, false, 2, false, 16)
// The same for the other long rows (k 8193-20480, e.g. 11008, 14336, 17408).
ZLM_GEMV_SKP(zlm_gemv_q6_k_r1_s5_sk2, Q6_K, 5, 2, 1, EPI_PLAIN, false, 2, false, 16)
ZLM_GEMV_SKP(zlm_gemv_q6_k_r1_s6_sk2, Q6_K, 6, 2, 1, EPI_PLAIN, false, 2, false, 16)
ZLM_GEMV_SKP(zlm_gemv_q6_k_r1_s7_sk2, Q6_K, 7, 2, 1, EPI_PLAIN, false, 2, false, 16)
ZLM_GEMV_SKP(zlm_gemv_q6_k_r1_s9_sk2, Q6_K, 9, 2, 1, EPI_PLAIN, false, 2, false, 16)
ZLM_GEMV_SKP(zlm_gemv_q6_k_r1_s10_sk2, Q6_K, 10, 2, 1, EPI_PLAIN, false, 2, false, 16)
ZLM_GEMV_SKP(zlm_gemv_q6_k_r1_s3_sk2, Q6_K, 3, 2, 1, EPI_PLAIN, false, 2, false, 16)
ZLM_GEMV_SKP(zlm_gemv_q6_k_r1_s4_sk2, Q6_K, 4, 2, 1, EPI_PLAIN, false, 2, false, 16)

ZLM_GEMV_MULTI_Q4(q6_k, Q6_K)

// Rows of 4097-8192 elements: the generic two-step loop over an 8192-element
// x tile, where the host takes it (measured faster than the exact-steps forms)
ZLM_GEMV_G8K(q6_k, Q6_K)
// The RMSNorm-fused lm_head at 3 chunk steps (from 65536 rows; the decode
// step's last op): the plain instance above with the norm prologue.  Measured
// on gfx950 (graph replays, weights rotated past the Infinity Cache): 152064 x
// 5120 191 -> 126 us against the 4-wave exact-steps instance.  At 2 steps the
// 4-wave normed instance already matches the plain lm_head instance (151936
// x 4096: 88.9 us both).
ZLM_GEMVX_PFQ(zlm_gemv_q6_k_norm_s3_tallq, Q6_K, 8192, 8, 2, 3, PRO_NORM, EPI_PLAIN, false)

// zlm_gemv_q4_0.hip -- the q4_0 GEMV entry points (plain and fused forms),
// built as their own gfx950 code object so the instance files compile in
// parallel.
#include "gemv_impl.h"

ZLM_GEMV_Q4(q4_0, Q4_0)
ZLM_GEMVX_Q4(q4_0, Q4_0)
ZLM_GEMVX_PAIR_TILES_Q4(q4_0, Q4_0)
ZLM_GEMVX_FORMS(q4_0, Q4_0, 16384, 6, true, s6)

// The residual form with two-row tiles, taken for launches of at most 8192
// rows at k <= 4096 (the decode step's o projection: 4.91 -> 4.54 us in the
// sweep harness, 1.619 -> 1.605 ms per decode token on gfx950).
ZLM_GEMVX(zlm_gemv_q4_0_resid_s2_r2, Q4_0, 4096, 2, 2, true, PRO_PLAIN, EPI_RESID)

// Prefetching forms for the decode-step shapes, x staged as int8 planes
// (v_dot4 on the nibbles), measured on gfx950 against the forms above:
// gate_up 12288 x 4096 with 8-wave workgroups at 8 waves per CU (16.3 ->
// 13.5 us in the sweep harness), down 4096 x 12288 with 16-wave workgroups at
// one per CU (10.4 -> 9.6 us), the normed q;k;v 6144 x 4096 with 8-wave
// workgroups at 16 waves per CU (6.4 -> 6.0 us).  4096-row launches (o, C0)
// stay plain: their workgroups have too few rows to repay the quantization.
// The normed gate_up runs 16-wave workgroups at one per CU (the RMSNorm and
// the planes are built once per 16 waves): decode step 1.6028 -> 1.5964 ms
// per token against 8-wave workgroups at 8 waves per CU.
ZLM_GEMVX_PFQ(zlm_gemv_q4_0_pair_s2_pfq, Q4_0, 4096, 8, 2, 2, PRO_PLAIN, EPI_PAIR, false)
ZLM_GEMVX_PFQ(zlm_gemv_q4_0_normpair_s2_pfqw16, Q4_0, 4096, 16, 2, 2, PRO_NORM, EPI_PAIR, false)
ZLM_GEMVX_PFQ(zlm_gemv_q4_0_resid_s6_pfqw16, Q4_0, 12288, 16, 1, 6, PRO_PLAIN, EPI_RESID, true)
ZLM_GEMVX_PFQ(zlm_gemv_q4_0_norm_s2_pfqw16, Q4_0, 4096, 8, 1, 2, PRO_NORM, EPI_PLAIN, false)

// Split-K forms of the down projection (k = 12288), x as int8 planes in
// registers: 6-wave workgroups, one per CU, four rows per tile.  Measured on
// gfx950 at 4096 x 12288 (resid): 9.6 us (resid_s6_pfqw16) -> 9.1 us.
ZLM_GEMV_SK(zlm_gemv_q4_0_r1_s6_sk4x, Q4_0, 6, 4, 1, EPI_PLAIN, true, 2, true)
ZLM_GEMV_SK(zlm_gemv_q4_0_resid_s6_sk4x, Q4_0, 6, 4, 1, EPI_RESID, true, 2, true)

// The same split-K forms for the other long rows (k 8193-20480: the FFN down
// projections of other models, e.g. k = 11008, 14336, 17408), any row of
// ceil(chunks / 64) == STEPS, one wave per chunk step.
ZLM_GEMV_SK(zlm_gemv_q4_0_r1_s5_sk4, Q4_0, 5, 4, 1, EPI_PLAIN, true, 2, false)
ZLM_GEMV_SK(zlm_gemv_q4_0_r1_s6_sk4, Q4_0, 6, 4, 1, EPI_PLAIN, true, 2, false)
ZLM_GEMV_SK(zlm_gemv_q4_0_r1_s7_sk4, Q4_0, 7, 4, 1, EPI_PLAIN, true, 2, false)
ZLM_GEMV_SK(zlm_gemv_q4_0_r1_s8_sk4, Q4_0, 8, 4, 1, EPI_PLAIN, true, 2, false)
ZLM_GEMV_SK(zlm_gemv_q4_0_r1_s9_sk4, Q4_0, 9, 4, 1, EPI_PLAIN, true, 2, false)
ZLM_GEMV_SK(zlm_gemv_q4_0_r1_s10_sk4, Q4_0, 10, 4, 1, EPI_PLAIN, true, 2, false)
ZLM_GEMV_SK(zlm_gemv_q4_0_resid_s5_sk4, Q4_0, 5, 4, 1, EPI_RESID, true, 2, false)
ZLM_GEMV_SK(zlm_gemv_q4_0_resid_s6_sk4, Q4_0, 6, 4, 1, EPI_RESID, true, 2, false)
ZLM_GEMV_SK(zlm_gemv_q4_0_resid_s7_sk4, Q4_0, 7, 4, 1, EPI_RESID, true, 2, false)
ZLM_GEMV_SK(zlm_gemv_q4_0_resid_s8_sk4, Q4_0, 8, 4, 1, EPI_RESID, true, 2, false)
ZLM_GEMV_SK(zlm_gemv_q4_0_resid_s9_sk4, Q4_0, 9, 4, 1, EPI_RESID, true, 2, false)
ZLM_GEMV_SK(zlm_gemv_q4_0_resid_s10_sk4, Q4_0, 10, 4, 1, EPI_RESID, true, 2, false)
ZLM_GEMV_SK(zlm_gemv_q4_0_r1_s3_sk4, Q4_0, 3, 4, 1, EPI_PLAIN, true, 2, false)
ZLM_GEMV_SK(zlm_gemv_q4_0_r1_s4_sk4, Q4_0, 4, 4, 1, EPI_PLAIN, true, 2, false)

ZLM_GEMV_MULTI_Q4(q4_0, Q4_0)

// matMul at m = 2 (both tokens in one pass over the weights)
ZLM_GEMV_TOK2(q4_0, Q4_0, 2)
ZLM_GEMVTR(zlm_gemv_q4_0_tok2_g4_r2, Q4_0, 4096, 4, 2, 2)
ZLM_GEMVTR(zlm_gemv_q4_0_tok2_g8_r2, Q4_0, 8192, 8, 2, 2)

// matMul at m = 3, 4 (int path, the weights read once for all tokens)
ZLM_GEMV_Q8TOK(q4_0, Q4_0, 2)
ZLM_GEMV_Q8TOK_R2(q4_0, Q4_0, 2)

// Rows of 4097-8192 elements: the generic two-step loop over an 8192-element
// x tile, where the host takes it (measured faster than the exact-steps forms)
ZLM_GEMV_G8K(q4_0, Q4_0)
// The lm_heads (from 65536 rows): prefetching 8-wave workgroups at 16 waves
// per CU with x as int8 planes, two-row wave tiles at 2-3 chunk steps (k <=
// 6144), one row at 4 (two hold too many registers).  Measured on gfx950
// against the 4-wave exact-steps instances (alternating runs, weights rotated
// past the Infinity Cache): 151936 x 4096 84 -> 62 us, 152064 x 5120 116 ->
// 88 us, 128256 x 8192 129 -> 102 us.
ZLM_GEMVX_PFQ(zlm_gemv_q4_0_r2_s2_tallq, Q4_0, 4096, 8, 2, 2, PRO_PLAIN, EPI_PLAIN, false)
ZLM_GEMVX_PFQ(zlm_gemv_q4_0_r2_s3_tallq, Q4_0, 8192, 8, 2, 3, PRO_PLAIN, EPI_PLAIN, false)
ZLM_GEMVX_PFQ(zlm_gemv_q4_0_r1_s4_tallq1, Q4_0, 8192, 8, 1, 4, PRO_PLAIN, EPI_PLAIN, false)
// The RMSNorm-fused lm_heads at 3-4 chunk steps (from 65536 rows).  Measured
// on gfx950 (graph replays, weights rotated past the Infinity Cache): 152064
// x 5120 110 -> 79 us, 128256 x 8192 121 -> 91.5 us.
ZLM_GEMVX_PFQ(zlm_gemv_q4_0_norm_s3_tallq, Q4_0, 8192, 8, 2, 3, PRO_NORM, EPI_PLAIN, false)
ZLM_GEMVX_PFQ(zlm_gemv_q4_0_norm_s4_tallq1, Q4_0, 8192, 8, 1, 4, PRO_NORM, EPI_PLAIN, false)

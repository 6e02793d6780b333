// zlm_gemv_q8_0.hip -- the q8_0 GEMV entry points (plain and fused forms),
// built as their own gfx950 code object so the instance files compile in
// parallel.
#include "gemv_impl.h"

ZLM_GEMV_Q8(q8_0, Q8_0)
ZLM_GEMVX_Q8(q8_0, Q8_0)
ZLM_GEMVX_PAIR_TILES_Q8(q8_0, Q8_0)

// Split-K form of the FFN down projection (k = 12288): 12-wave workgroups,
// one per CU, each wave one chunk step of two rows per tile.  Measured on
// gfx950 at 4096 x 12288: 13.1 -> 10.5 us (the one-wave-per-row kernel takes
// ~320 registers per wave and runs one wave per SIMD).
ZLM_GEMV_SK(zlm_gemv_q8_0_r1_s12_sk2x, Q8_0, 12, 2, 1, EPI_PLAIN, false, 2, true)

// The same for the other long rows (k 8193-20480, e.g. 11008, 14336, 17408),
// any row of ceil(chunks / 64) == STEPS: one wave per chunk step up to 16
// steps, two steps per wave beyond (17 steps take the 18-step workgroup).
ZLM_GEMV_SK(zlm_gemv_q8_0_r1_s9_sk2, Q8_0, 9, 2, 1, EPI_PLAIN, false, 2, false)
ZLM_GEMV_SK(zlm_gemv_q8_0_r1_s10_sk2, Q8_0, 10, 2, 1, EPI_PLAIN, false, 2, false)
ZLM_GEMV_SK(zlm_gemv_q8_0_r1_s11_sk2, Q8_0, 11, 2, 1, EPI_PLAIN, false, 2, false)
ZLM_GEMV_SK(zlm_gemv_q8_0_r1_s12_sk2, Q8_0, 12, 2, 1, EPI_PLAIN, false, 2, false)
ZLM_GEMV_SK(zlm_gemv_q8_0_r1_s13_sk2, Q8_0, 13, 2, 1, EPI_PLAIN, false, 2, false)
ZLM_GEMV_SK(zlm_gemv_q8_0_r1_s14_sk2, Q8_0, 14, 2, 1, EPI_PLAIN, false, 2, false)
ZLM_GEMV_SK(zlm_gemv_q8_0_r1_s15_sk2, Q8_0, 15, 2, 1, EPI_PLAIN, false, 2, false)
ZLM_GEMV_SK(zlm_gemv_q8_0_r1_s16_sk2, Q8_0, 16, 2, 1, EPI_PLAIN, false, 2, false)
ZLM_GEMV_SK(zlm_gemv_q8_0_r1_s17_sk2, Q8_0, 9, 2, 2, EPI_PLAIN, false, 2, false)
ZLM_GEMV_SK(zlm_gemv_q8_0_r1_s18_sk2, Q8_0, 9, 2, 2, EPI_PLAIN, false, 2, false)
ZLM_GEMV_SK(zlm_gemv_q8_0_r1_s19_sk2, Q8_0, 10, 2, 2, EPI_PLAIN, false, 2, false)
ZLM_GEMV_SK(zlm_gemv_q8_0_r1_s20_sk2, Q8_0, 10, 2, 2, EPI_PLAIN, false, 2, false)
ZLM_GEMV_SK(zlm_gemv_q8_0_r1_s5_sk2, Q8_0, 5, 2, 1, EPI_PLAIN, false, 2, false)
ZLM_GEMV_SK(zlm_gemv_q8_0_r1_s6_sk2, Q8_0, 6, 2, 1, EPI_PLAIN, false, 2, false)
ZLM_GEMV_SK(zlm_gemv_q8_0_r1_s7_sk2, Q8_0, 7, 2, 1, EPI_PLAIN, false, 2, false)
ZLM_GEMV_SK(zlm_gemv_q8_0_r1_s8_sk2, Q8_0, 8, 2, 1, EPI_PLAIN, false, 2, false)

// Exact-steps instances for k = 5120 and 7168 (hidden sizes of other models).
ZLM_GEMV(zlm_gemv_q8_0_r1_s5, Q8_0, 8192, 1, 5, true)
ZLM_GEMV(zlm_gemv_q8_0_r1_s7, Q8_0, 8192, 1, 7, true)

// The lm_heads (from 65536 rows, k = 4096): prefetching 8-wave workgroups at
// 16 waves per CU, plain and RMSNorm-fused; measured on gfx950 at 151936 x
// 4096: 98.6 -> 94.8 us against the 4-wave exact-steps instance at 8
// workgroups per CU.
ZLM_GEMVX_PF(zlm_gemv_q8_0_r1_s4_tall, Q8_0, 4096, 8, 1, 4, PRO_PLAIN, EPI_PLAIN, false)
ZLM_GEMVX_PF(zlm_gemv_q8_0_norm_s4_tall, Q8_0, 4096, 8, 1, 4, PRO_NORM, EPI_PLAIN, false)

ZLM_GEMV_MULTI_Q8(q8_0, Q8_0)

// matMul at m = 2 (both tokens in one pass over the weights)
ZLM_GEMV_TOK2(q8_0, Q8_0, 4)
ZLM_GEMVTR(zlm_gemv_q8_0_tok2_g4_r2, Q8_0, 4096, 4, 2, 4)
ZLM_GEMVTR(zlm_gemv_q8_0_tok2_g8_r2, Q8_0, 8192, 8, 2, 4)

// matMul at m = 3, 4 (int path, the weights read once for all tokens)
ZLM_GEMV_Q8TOK(q8_0, Q8_0, 4)
// The lm_heads at 5-8 chunk steps (k 4097-8192, from 65536 rows): the
// prefetching 8-wave instance of the 4-step lm_head; at 7-8 steps with
// scheduling fences (without them the 8-step form spills).  Measured on
// gfx950 against the exact-steps and generic instances (alternating runs,
// weights rotated past the Infinity Cache): 152064 x 5120 179 -> 129 us,
// 65536 x 5120 81 -> 59 us, 151936 x 6144 232 -> 155 us, 151936 x 7168 200 ->
// 181 us, 128256 x 8192 184 -> 172 us.
ZLM_GEMVX_PF(zlm_gemv_q8_0_r1_s5_tall, Q8_0, 8192, 8, 1, 5, PRO_PLAIN, EPI_PLAIN, false)
ZLM_GEMVX_PF(zlm_gemv_q8_0_r1_s6_tall, Q8_0, 8192, 8, 1, 6, PRO_PLAIN, EPI_PLAIN, false)
ZLM_GEMVX_PF(zlm_gemv_q8_0_r1_s7_tall, Q8_0, 8192, 8, 1, 7, PRO_PLAIN, EPI_PLAIN, true)
ZLM_GEMVX_PF(zlm_gemv_q8_0_r1_s8_tall, Q8_0, 8192, 8, 1, 8, PRO_PLAIN, EPI_PLAIN, true)
// The RMSNorm-fused lm_heads at 5-8 chunk steps (from 65536 rows): the
// instances above with the norm prologue.  Measured on gfx950 (graph
// replays, weights rotated past the Infinity Cache): 152064 x 5120 240 -> 123
// us (the generic instance before), 128256 x 8192 177 -> 169 us.
ZLM_GEMVX_PF(zlm_gemv_q8_0_norm_s5_tall, Q8_0, 8192, 8, 1, 5, PRO_NORM, EPI_PLAIN, false)
ZLM_GEMVX_PF(zlm_gemv_q8_0_norm_s6_tall, Q8_0, 8192, 8, 1, 6, PRO_NORM, EPI_PLAIN, false)
ZLM_GEMVX_PF(zlm_gemv_q8_0_norm_s7_tall, Q8_0, 8192, 8, 1, 7, PRO_NORM, EPI_PLAIN, true)
ZLM_GEMVX_PF(zlm_gemv_q8_0_norm_s8_tall, Q8_0, 8192, 8, 1, 8, PRO_NORM, EPI_PLAIN, true)

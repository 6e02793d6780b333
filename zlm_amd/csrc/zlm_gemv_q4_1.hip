// zlm_gemv_q4_1.hip -- the q4_1 GEMV entry points (plain and fused forms),
// built as their own gfx950 code object so the instance files compile in
// parallel.
#include "gemv_impl.h"

ZLM_GEMV_Q4_COMMON(q4_1, Q4_1)
ZLM_GEMVX_Q4(q4_1, Q4_1)
ZLM_GEMVX_PAIR_TILES_Q4(q4_1, Q4_1)

ZLM_GEMV_MULTI_Q4(q4_1, Q4_1)

// matMul at m = 2 (both tokens in one pass over the weights)
ZLM_GEMV_TOK2(q4_1, Q4_1, 2)
ZLM_GEMVTR(zlm_gemv_q4_1_tok2_g4_r2, Q4_1, 4096, 4, 2, 2)
ZLM_GEMVTR(zlm_gemv_q4_1_tok2_g8_r2, Q4_1, 8192, 8, 2, 2)

// matMul at m = 3, 4 (int path, the weights read once for all tokens)
ZLM_GEMV_Q8TOK(q4_1, Q4_1, 2)
ZLM_GEMV_Q8TOK8(q4_1, Q4_1, 2)
ZLM_GEMV_Q8TOK16(q4_1, Q4_1, 2)
ZLM_GEMV_Q8TOK_R2(q4_1, Q4_1, 2)

// Rows of 4097-8192 elements: the generic two-step loop over an 8192-element
// x tile, where the host takes it (measured faster than the exact-steps forms)
ZLM_GEMV_G8K(q4_1, Q4_1)
// The lm_heads (from 65536 rows): prefetching 8-wave workgroups at 16 waves
// per CU (fp32 x).  Measured on gfx950 against the exact-steps instances
// (alternating runs, weights rotated past the Infinity Cache): 151936 x 4096
// 87 -> 84 us, 152064 x 5120 117 -> 110 us, 128256 x 8192 134 -> 128 us.
ZLM_GEMVX_PF(zlm_gemv_q4_1_r1_s2_tall, Q4_1, 4096, 8, 1, 2, PRO_PLAIN, EPI_PLAIN, false)
ZLM_GEMVX_PF(zlm_gemv_q4_1_r1_s3_tall, Q4_1, 8192, 8, 1, 3, PRO_PLAIN, EPI_PLAIN, false)
ZLM_GEMVX_PF(zlm_gemv_q4_1_r1_s4_tall, Q4_1, 8192, 8, 1, 4, PRO_PLAIN, EPI_PLAIN, false)
// The RMSNorm-fused lm_heads at 3-4 chunk steps (from 65536 rows).  Measured
// on gfx950 (graph replays, weights rotated past the Infinity Cache): 152064
// x 5120 112 -> 101 us, 128256 x 8192 125 -> 117 us.
ZLM_GEMVX_PF(zlm_gemv_q4_1_norm_s3_tall, Q4_1, 8192, 8, 1, 3, PRO_NORM, EPI_PLAIN, false)
ZLM_GEMVX_PF(zlm_gemv_q4_1_norm_s4_tall, Q4_1, 8192, 8, 1, 4, PRO_NORM, EPI_PLAIN, false)

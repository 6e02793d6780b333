// zlm_gemv_q6_k.hip -- the q6_k GEMV entry points (plain and fused forms),
// built as their own gfx950 code object so the instance files compile in
// parallel.
#include "gemv_impl.h"

ZLM_GEMV_Q4_COMMON(q6_k, Q6_K)
ZLM_GEMVX_Q4(q6_k, Q6_K)

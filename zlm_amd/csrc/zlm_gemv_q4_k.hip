// zlm_gemv_q4_k.hip -- the q4_k GEMV entry points (plain and fused forms),
// built as their own gfx950 code object so the instance files compile in
// parallel.
#include "gemv_impl.h"

ZLM_GEMV_Q4_COMMON(q4_k, Q4_K)
ZLM_GEMVX_Q4(q4_k, Q4_K)

// zlm_gemv_q8_0.hip -- the q8_0 GEMV entry points (plain and fused forms),
// built as their own gfx950 code object so the instance files compile in
// parallel.
#include "gemv_impl.h"

ZLM_GEMV_Q8(q8_0, Q8_0)
ZLM_GEMVX_Q8(q8_0, Q8_0)

ZLM_GEMV_MULTI_Q8(q8_0, Q8_0)

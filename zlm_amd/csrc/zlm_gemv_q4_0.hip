// zlm_gemv_q4_0.hip -- the q4_0 GEMV entry points (plain and fused forms),
// built as their own gfx950 code object so the instance files compile in
// parallel.
#include "gemv_impl.h"

ZLM_GEMV_Q4(q4_0, Q4_0)
ZLM_GEMVX_Q4(q4_0, Q4_0)
ZLM_GEMVX_FORMS(q4_0, Q4_0, 16384, 6, true, s6)

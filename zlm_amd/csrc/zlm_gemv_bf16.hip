// zlm_gemv_bf16.hip -- the bf16 GEMV entry points (plain and fused forms),
// built as their own gfx950 code object so the instance files compile in
// parallel.
#include "gemv_impl.h"

ZLM_GEMV_F16(bf16, BF16)
ZLM_GEMVX_F16(bf16, BF16)

ZLM_GEMV_MULTI_F16(bf16, BF16)

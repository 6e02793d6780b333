// zlm_gemv_f32.hip -- the f32 GEMV entry points (plain and fused forms),
// built as their own gfx950 code object so the instance files compile in
// parallel.
#include "gemv_impl.h"

ZLM_GEMV_F32(f32, F32)
ZLM_GEMVX_F32(f32, F32)

ZLM_GEMV_MULTI_F32(f32, F32)

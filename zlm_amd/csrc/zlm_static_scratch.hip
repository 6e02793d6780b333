// The fixed device scratch behind zlm_gpu_attention_decode_enqueue_noalloc:
// a file-scope device array, so the entry point needs no allocation at any
// call (it may be captured into a HIP graph first, or run where hipMalloc is
// not allowed).  Compiled by hipcc into the host library; the array lives in
// this object's gfx950 code object and is loaded with it.
#include "zlm_static_scratch.h"

#include <hip/hip_runtime.h>

static __device__ __align__(256) float scratch[ZLM_STATIC_SCRATCH_FLOATS];

hipError_t zlm_static_scratch_address(float** ptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    *ptr = e == hipSuccess ? static_cast<float*>(p) : nullptr;
    return e;
}

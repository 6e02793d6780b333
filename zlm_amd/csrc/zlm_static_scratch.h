// Internal interface of zlm_static_scratch.hip: the fixed device scratch of the
// entry points that allocate nothing.
#ifndef ZLM_STATIC_SCRATCH_H
#define ZLM_STATIC_SCRATCH_H

#include <stddef.h>

#include <hip/hip_runtime_api.h>

// Floats in the array: 16384 attention head-splits (one q head over one
// 64-position range) of 130 floats each (128 unnormalised outputs, the split's
// max score and its exp-sum), 8,519,680 bytes.
#define ZLM_STATIC_SCRATCH_HEAD_SPLITS 16384u
#define ZLM_STATIC_SCRATCH_FLOATS (ZLM_STATIC_SCRATCH_HEAD_SPLITS * 130u)

// Device address of the current device's copy of the array (each GPU holds its
// own copy at its own address).  Call once per device, with that device
// current; the host-side name of the array is not a device address.
hipError_t zlm_static_scratch_address(float** ptr);

#endif

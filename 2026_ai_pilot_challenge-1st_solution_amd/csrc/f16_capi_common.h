// f16_capi_common.h -- return-code conventions shared by the C entry points.
//   0              success
//   F16_EINVAL     bad size, stride or null pointer (nothing launched)
//   F16_ERATE      unsupported FCS component rate (nothing launched)
//   -(1000 + e)    HIP runtime error e from the launch
#pragma once
#include <hip/hip_runtime.h>

#define F16_EINVAL (-1)
#define F16_ERATE (-2)
#define F16_ETOOBIG (-3)

static inline int f16_last_error(void) {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : -(1000 + (int)e);
}

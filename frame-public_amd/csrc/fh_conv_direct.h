// Conv2d definitions of the direct (NCHW) path: geometry and the per-element elementwise epilogue.
#pragma once

#include <hip/hip_runtime.h>

#include "fh_common.h"

namespace fh {

struct ConvGeom {
  int64_t n, cin, h, w, cout, kh, kw, sh, sw, ph, pw, groups, oh, ow;
};

struct ConvEpilogue {
  int32_t nseg;
  int32_t round_between;
  uint8_t ops[FH_MAX_SEGMENTS];
  const void* ins[FH_MAX_SEGMENTS];
};

// Runs the epilogue program on one rounded conv output value at flat output index `idx` (NCHW).
template <typename T>
__device__ __forceinline__ float conv_epilogue(const ConvEpilogue& ep, float v, int64_t idx) {
  return epilogue_one<T>(ep, v, idx);
}

}  // namespace fh

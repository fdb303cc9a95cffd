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
  using S = typename Io<T>::storage;
  for (int s = 0; s < ep.nseg; ++s) {
    const uint8_t op = ep.ops[s];
    if (ew_is_binary(op)) {
      v = ew_binary(op, v, Io<T>::load(static_cast<const S*>(ep.ins[s])[idx]));
    } else {
      v = ew_unary(op, v);
    }
    if (ep.round_between) v = Io<T>::round(v);
  }
  return v;
}

}  // namespace fh

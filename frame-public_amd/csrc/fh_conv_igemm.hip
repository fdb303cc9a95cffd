// Implicit-GEMM conv2d on MFMA (placeholder selection: not yet enabled for any shape).
#include "fh_conv_igemm.h"

namespace fh {

template <typename T>
bool conv_igemm_supported(const ConvGeom&, const void*, const void*, const void*, const ConvEpilogue&) {
  return false;
}

template <typename T>
fh_status conv_igemm_launch(const void*, const void*, const void*, void*, const ConvGeom&, const ConvEpilogue&,
                            hipStream_t) {
  return fail(FH_UNIMPLEMENTED, "conv implicit GEMM not available for this shape");
}

template bool conv_igemm_supported<float>(const ConvGeom&, const void*, const void*, const void*,
                                          const ConvEpilogue&);
template bool conv_igemm_supported<bf16_t>(const ConvGeom&, const void*, const void*, const void*,
                                           const ConvEpilogue&);
template bool conv_igemm_supported<f16_t>(const ConvGeom&, const void*, const void*, const void*,
                                          const ConvEpilogue&);
template fh_status conv_igemm_launch<float>(const void*, const void*, const void*, void*, const ConvGeom&,
                                            const ConvEpilogue&, hipStream_t);
template fh_status conv_igemm_launch<bf16_t>(const void*, const void*, const void*, void*, const ConvGeom&,
                                             const ConvEpilogue&, hipStream_t);
template fh_status conv_igemm_launch<f16_t>(const void*, const void*, const void*, void*, const ConvGeom&,
                                            const ConvEpilogue&, hipStream_t);

}  // namespace fh

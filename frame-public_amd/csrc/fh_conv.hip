// Conv2d forward, NCHW (reference semantics: src/backends/cpu/kernels/conv.cpp:223-314).
//
// conv2d_direct_kernel: one thread per output element, products summed over (ci, kh, kw) in the reference's
// order, bias added last inside the fp32 accumulator, one rounding. It serves every geometry (groups,
// strides, padding, odd channel counts, fp32) on NCHW operands. The MFMA implicit-GEMM path over
// channels-last operands is fh_conv2d_nhwc_fwd (fh_conv_igemm.hip), selected at graph compile time.
#include <hip/hip_runtime.h>

#include <string>

#include "fh_common.h"
#include "fh_conv_direct.h"

namespace fh {
namespace {

template <typename T>
__global__ __launch_bounds__(256) void conv2d_direct_kernel(const typename Io<T>::storage* __restrict__ x,
                                                            const typename Io<T>::storage* __restrict__ w,
                                                            const typename Io<T>::storage* __restrict__ bias,
                                                            typename Io<T>::storage* __restrict__ y, ConvGeom g,
                                                            ConvEpilogue ep) {
  using S = typename Io<T>::storage;
  const int64_t total = g.n * g.cout * g.oh * g.ow;
  const int64_t cin_g = g.cin / g.groups;
  const int64_t cout_g = g.cout / g.groups;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t ow = i % g.ow;
    const int64_t oh = (i / g.ow) % g.oh;
    const int64_t co = (i / (g.ow * g.oh)) % g.cout;
    const int64_t n = i / (g.ow * g.oh * g.cout);
    const int64_t grp = co / cout_g;
    float acc = 0.0f;
    for (int64_t ci = 0; ci < cin_g; ++ci) {
      const S* xp = x + ((n * g.cin + grp * cin_g + ci) * g.h) * g.w;
      const S* wp = w + ((co * cin_g + ci) * g.kh) * g.kw;
      for (int64_t a = 0; a < g.kh; ++a) {
        const int64_t ih = oh * g.sh - g.ph + a;
        if (ih < 0 || ih >= g.h) continue;
        for (int64_t b = 0; b < g.kw; ++b) {
          const int64_t iw = ow * g.sw - g.pw + b;
          if (iw < 0 || iw >= g.w) continue;
          acc += Io<T>::load(xp[ih * g.w + iw]) * Io<T>::load(wp[a * g.kw + b]);
        }
      }
    }
    if (bias != nullptr) acc += Io<T>::load(bias[co]);
    y[i] = Io<T>::store(conv_epilogue<T>(ep, Io<T>::round(acc), i));
  }
}

template <typename T>
fh_status launch_direct(const void* x, const void* w, const void* bias, void* y, const ConvGeom& g,
                        const ConvEpilogue& ep, hipStream_t s) {
  using S = typename Io<T>::storage;
  const int64_t total = g.n * g.cout * g.oh * g.ow;
  int64_t blocks = (total + 255) / 256;
  const int64_t cap = static_cast<int64_t>(device_cu_count()) * 32;
  if (blocks > cap) blocks = cap;
  hipLaunchKernelGGL((conv2d_direct_kernel<T>), dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, s,
                     static_cast<const S*>(x), static_cast<const S*>(w), static_cast<const S*>(bias),
                     static_cast<S*>(y), g, ep);
  return launch_status("conv2d_direct_kernel launch");
}

template <typename T>
fh_status conv_typed(const void* x, const void* w, const void* bias, void* y, const ConvGeom& g,
                     const ConvEpilogue& ep, hipStream_t s) {
  return launch_direct<T>(x, w, bias, y, g, ep, s);
}

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" fh_status fh_conv2d_fwd(int32_t dtype, const void* x, const void* w, const void* bias, void* y,
                                   const int64_t geom[12], const fh_epilogue* epilogue, void* stream) {
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, "fh_conv2d_fwd: unsupported dtype");
  if (geom == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_conv2d_fwd: null geometry");
  ConvGeom g{};
  g.n = geom[0];
  g.cin = geom[1];
  g.h = geom[2];
  g.w = geom[3];
  g.cout = geom[4];
  g.kh = geom[5];
  g.kw = geom[6];
  g.sh = geom[7];
  g.sw = geom[8];
  g.ph = geom[9];
  g.pw = geom[10];
  g.groups = geom[11];
  if (g.n < 0 || g.cin <= 0 || g.h < 0 || g.w < 0 || g.cout <= 0 || g.kh <= 0 || g.kw <= 0 || g.sh <= 0 ||
      g.sw <= 0 || g.ph < 0 || g.pw < 0 || g.groups <= 0)
    return fail(FH_INVALID_ARGUMENT, "fh_conv2d_fwd: invalid geometry");
  if (g.cin % g.groups != 0 || g.cout % g.groups != 0)
    return fail(FH_INVALID_ARGUMENT, "fh_conv2d_fwd: channels not divisible by groups");
  if (g.h + 2 * g.ph < g.kh || g.w + 2 * g.pw < g.kw)
    return fail(FH_INVALID_ARGUMENT, "fh_conv2d_fwd: kernel larger than the padded input");
  g.oh = (g.h + 2 * g.ph - g.kh) / g.sh + 1;
  g.ow = (g.w + 2 * g.pw - g.kw) / g.sw + 1;
  ConvEpilogue ep{};
  if (epilogue != nullptr) {
    if (epilogue->nseg < 0 || epilogue->nseg > FH_MAX_SEGMENTS)
      return fail(FH_INVALID_ARGUMENT, "fh_conv2d_fwd: epilogue nseg out of range");
    ep.nseg = epilogue->nseg;
    ep.round_between = epilogue->round_between;
    for (int s = 0; s < ep.nseg; ++s) {
      if (!epilogue_op_ok(epilogue->ops[s]))
        return fail(FH_INVALID_ARGUMENT, "fh_conv2d_fwd: unknown epilogue op");
      if (ew_is_binary(epilogue->ops[s]) && epilogue->ins[s] == nullptr)
        return fail(FH_INVALID_ARGUMENT, "fh_conv2d_fwd: binary epilogue segment without operand");
      ep.ops[s] = epilogue->ops[s];
      ep.ins[s] = epilogue->ins[s];
    }
  }
  if (g.n * g.cout * g.oh * g.ow == 0) return FH_OK;
  if (x == nullptr || w == nullptr || y == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_conv2d_fwd: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case FH_F32:
      return conv_typed<float>(x, w, bias, y, g, ep, s);
    case FH_BF16:
      return conv_typed<bf16_t>(x, w, bias, y, g, ep, s);
    default:
      return conv_typed<f16_t>(x, w, bias, y, g, ep, s);
  }
}

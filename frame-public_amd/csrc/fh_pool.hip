// 2-D pooling over NCHW, one thread per output element (the operation is a small gather; its cost is the
// read of the input once and the write of the output once). The per-plane kernel keeps index math in 32 bits.
//
// max_pool2d (reference: src/backends/cpu/kernels/pool.cpp:178-237): padding never wins (treated as -inf),
// the window is scanned kh-outer / kw-inner and a later value replaces the best only if strictly greater,
// so the first maximum wins. A window without any valid position is rejected on the host.
// avg_pool2d (reference: src/backends/cpu/kernels/pool.cpp:283-306): padding counts as zero, the
// denominator is always KH*KW.
#include <hip/hip_runtime.h>

#include <string>

#include "fh_common.h"

namespace fh {
namespace {

struct PoolGeom {
  int64_t n, c, h, w, kh, kw, sh, sw, ph, pw, oh, ow;
};

template <typename T, int MODE>
__global__ __launch_bounds__(256) void pool2d_kernel(const typename Io<T>::storage* __restrict__ x,
                                                     typename Io<T>::storage* __restrict__ y, PoolGeom g) {
  const int64_t total = g.n * g.c * g.oh * g.ow;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const float denom = static_cast<float>(g.kh * g.kw);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t ow = i % g.ow;
    const int64_t oh = (i / g.ow) % g.oh;
    const int64_t nc = i / (g.ow * g.oh);
    const auto* plane = x + nc * g.h * g.w;
    float acc = 0.0f;
    bool found = false;
    for (int64_t a = 0; a < g.kh; ++a) {
      const int64_t ih = oh * g.sh - g.ph + a;
      if (ih < 0 || ih >= g.h) continue;
      for (int64_t b = 0; b < g.kw; ++b) {
        const int64_t iw = ow * g.sw - g.pw + b;
        if (iw < 0 || iw >= g.w) continue;
        const float v = Io<T>::load(plane[ih * g.w + iw]);
        if (MODE == 0) {
          if (!found || v > acc) acc = v;
          found = true;
        } else {
          acc += v;
        }
      }
    }
    y[i] = Io<T>::store(MODE == 0 ? acc : acc / denom);
  }
}

// Same semantics with one grid row per (image, channel) plane and 32-bit index math inside the plane (the 64-bit
// divisions of the general kernel dominate its run time). Used when a plane has fewer than 2^31 elements and
// there are at most 65535 * 65535 planes' worth of grid.
struct PlaneGeom {
  int32_t h, w, kh, kw, sh, sw, ph, pw, oh, ow;
};

template <typename T, int MODE>
__global__ __launch_bounds__(256) void pool2d_plane_kernel(const typename Io<T>::storage* __restrict__ x,
                                                           typename Io<T>::storage* __restrict__ y, PlaneGeom g) {
  const int p = blockIdx.x * 256 + threadIdx.x;
  const int ohw = g.oh * g.ow;
  if (p >= ohw) return;
  const int64_t plane_id = static_cast<int64_t>(blockIdx.z) * gridDim.y + blockIdx.y;
  const int oh = p / g.ow, ow = p - (p / g.ow) * g.ow;
  const auto* plane = x + plane_id * g.h * g.w;
  const float denom = static_cast<float>(g.kh * g.kw);
  float acc = 0.0f;
  bool found = false;
  const int ih0 = oh * g.sh - g.ph, iw0 = ow * g.sw - g.pw;
  for (int a = 0; a < g.kh; ++a) {
    const int ih = ih0 + a;
    if (ih < 0 || ih >= g.h) continue;
    const auto* rowp = plane + ih * g.w;
    for (int b = 0; b < g.kw; ++b) {
      const int iw = iw0 + b;
      if (iw < 0 || iw >= g.w) continue;
      const float v = Io<T>::load(rowp[iw]);
      if (MODE == 0) {
        if (!found || v > acc) acc = v;
        found = true;
      } else {
        acc += v;
      }
    }
  }
  y[plane_id * ohw + p] = Io<T>::store(MODE == 0 ? acc : acc / denom);
}

template <typename T>
fh_status launch_pool(int32_t mode, const void* x, void* y, const PoolGeom& g, hipStream_t s) {
  using S = typename Io<T>::storage;
  const int64_t planes = g.n * g.c;
  if (g.h * g.w < (int64_t{1} << 31) && g.oh * g.ow < (int64_t{1} << 31) && planes <= int64_t{65535} * 65535) {
    const PlaneGeom pg{static_cast<int32_t>(g.h),  static_cast<int32_t>(g.w),  static_cast<int32_t>(g.kh),
                       static_cast<int32_t>(g.kw), static_cast<int32_t>(g.sh), static_cast<int32_t>(g.sw),
                       static_cast<int32_t>(g.ph), static_cast<int32_t>(g.pw), static_cast<int32_t>(g.oh),
                       static_cast<int32_t>(g.ow)};
    // planes = gy * gz exactly: gy the largest divisor of planes not above 65535
    int64_t gy = planes <= 65535 ? planes : 65535;
    while (planes % gy != 0) --gy;
    const int64_t gz = planes / gy;
    if (gz <= 65535) {
      const dim3 grid(static_cast<uint32_t>((g.oh * g.ow + 255) / 256), static_cast<uint32_t>(gy), static_cast<uint32_t>(gz));
      if (mode == 0) {
        hipLaunchKernelGGL((pool2d_plane_kernel<T, 0>), grid, dim3(256), 0, s, static_cast<const S*>(x), static_cast<S*>(y), pg);
      } else {
        hipLaunchKernelGGL((pool2d_plane_kernel<T, 1>), grid, dim3(256), 0, s, static_cast<const S*>(x), static_cast<S*>(y), pg);
      }
      return launch_status("pool2d_plane_kernel launch");
    }
  }
  const int64_t total = g.n * g.c * g.oh * g.ow;
  int64_t blocks = (total + 255) / 256;
  const int64_t cap = static_cast<int64_t>(device_cu_count()) * 16;
  if (blocks > cap) blocks = cap;
  if (mode == 0) {
    hipLaunchKernelGGL((pool2d_kernel<T, 0>), dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, s,
                       static_cast<const S*>(x), static_cast<S*>(y), g);
  } else {
    hipLaunchKernelGGL((pool2d_kernel<T, 1>), dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, s,
                       static_cast<const S*>(x), static_cast<S*>(y), g);
  }
  return launch_status("pool2d_kernel launch");
}

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" fh_status fh_pool2d(int32_t dtype, int32_t mode, const void* x, void* y, const int64_t geom[10],
                               void* stream) {
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, "fh_pool2d: unsupported dtype");
  if (mode != 0 && mode != 1) return fail(FH_INVALID_ARGUMENT, "fh_pool2d: mode must be 0 (max) or 1 (avg)");
  if (geom == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_pool2d: null geometry");
  PoolGeom g{geom[0], geom[1], geom[2], geom[3], geom[4], geom[5], geom[6], geom[7], geom[8], geom[9], 0, 0};
  if (g.n < 0 || g.c < 0 || g.h < 0 || g.w < 0 || g.kh <= 0 || g.kw <= 0 || g.sh <= 0 || g.sw <= 0 || g.ph < 0 ||
      g.pw < 0)
    return fail(FH_INVALID_ARGUMENT, "fh_pool2d: invalid geometry");
  if (g.h + 2 * g.ph < g.kh || g.w + 2 * g.pw < g.kw)
    return fail(FH_INVALID_ARGUMENT, "fh_pool2d: window larger than the padded input");
  g.oh = (g.h + 2 * g.ph - g.kh) / g.sh + 1;
  g.ow = (g.w + 2 * g.pw - g.kw) / g.sw + 1;
  if (mode == 0) {
    // Every window must hold a valid position: the last window start must not lie beyond the input and the
    // first window must reach into it (reference rejects such windows with kInternal).
    if (g.ph >= g.kh || g.pw >= g.kw || (g.oh - 1) * g.sh - g.ph >= g.h || (g.ow - 1) * g.sw - g.pw >= g.w)
      return fail(FH_INVALID_ARGUMENT, "fh_pool2d: a max-pool window has no valid (non-padding) position");
  }
  if (g.n * g.c * g.oh * g.ow == 0) return FH_OK;
  if (x == nullptr || y == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_pool2d: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case FH_F32:
      return launch_pool<float>(mode, x, y, g, s);
    case FH_BF16:
      return launch_pool<bf16_t>(mode, x, y, g, s);
    default:
      return launch_pool<f16_t>(mode, x, y, g, s);
  }
}

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

// Max pool 3x3, stride 2, padding 1 on 16-bit data (ResNet's stem pool), W % 16 == 0: one thread per 8
// consecutive outputs of a row. Each of the 3 input rows is read as two 16-byte vectors (columns 2*ow0 ..
// 2*ow0 + 15) plus the element left of them, and every window is scanned in the general kernel's order
// (kh outer, kw inner, strictly greater replaces), so the selected values are the same bits.
template <typename T>
__global__ __launch_bounds__(256) void maxpool3s2_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                         int32_t h, int32_t w, int32_t oh, int32_t ow, int32_t total) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int qn = ow / 8;
  const int q = idx % qn, t2 = idx / qn;
  const int o_h = t2 % oh;
  const int64_t plane = t2 / oh;
  const int c0 = 16 * q;  // first input column of the 8 windows' centres - 1 ... (2 * ow0)
  const uint16_t* px = x + plane * h * w;
  float acc[8];
  bool found[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    acc[j] = 0.0f;
    found[j] = false;
  }
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    const int ih = 2 * o_h - 1 + a;
    if (ih < 0 || ih >= h) continue;
    const uint16_t* row = px + static_cast<int64_t>(ih) * w + c0;
    const uint4 v0 = *reinterpret_cast<const uint4*>(row);
    const uint4 v1 = *reinterpret_cast<const uint4*>(row + 8);
    uint16_t e[17];  // e[0] = column c0 - 1, e[1 + k] = column c0 + k
    __builtin_memcpy(e + 1, &v0, 16);
    __builtin_memcpy(e + 9, &v1, 16);
    const bool left = c0 > 0;
    e[0] = left ? row[-1] : uint16_t{0};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int b = 0; b < 3; ++b) {
        const int k = 2 * j + b;  // index into e: column c0 + 2j - 1 + b
        if (k == 0 && !left) continue;
        const float v = Io<T>::load(e[k]);
        if (!found[j] || v > acc[j]) acc[j] = v;
        found[j] = true;
      }
    }
  }
  uint16_t o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = Io<T>::store(acc[j]);
  uint4 out;
  __builtin_memcpy(&out, o, 16);
  *reinterpret_cast<uint4*>(y + (plane * oh + o_h) * ow + 8 * q) = out;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <typename T>
fh_status launch_pool(int32_t mode, const void* x, void* y, const PoolGeom& g, hipStream_t s) {
  using S = typename Io<T>::storage;
  const int64_t planes = g.n * g.c;
  if constexpr (sizeof(S) == 2) {
    const int64_t total = planes * g.oh * (g.ow / 8);
    if (mode == 0 && g.kh == 3 && g.kw == 3 && g.sh == 2 && g.sw == 2 && g.ph == 1 && g.pw == 1 && g.w % 16 == 0 &&
        g.ow % 8 == 0 && g.ow * 2 == g.w && aligned16(x) && aligned16(y) && total < (int64_t{1} << 31)) {
      hipLaunchKernelGGL((maxpool3s2_kernel<T>), dim3(static_cast<uint32_t>((total + 255) / 256)), dim3(256), 0, s,
                         static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), static_cast<int32_t>(g.h),
                         static_cast<int32_t>(g.w), static_cast<int32_t>(g.oh), static_cast<int32_t>(g.ow),
                         static_cast<int32_t>(total));
      return launch_status("maxpool3s2_kernel launch");
    }
  }
  // per-plane grid rows only when a plane fills most of a 256-thread block (a global pool would idle 255 of 256)
  if (g.oh * g.ow >= 192 && g.h * g.w < (int64_t{1} << 31) && g.oh * g.ow < (int64_t{1} << 31) &&
      planes <= int64_t{65535} * 65535) {
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

// Channels-last pooling, x [N][H][W][C] -> y [N][Ho][Wo][C]: one thread per output pixel and group of VW
// consecutive channels (one 16-byte vector when C allows, else VW = 1), each channel with the NCHW kernel's
// semantics and scan order. 32-bit index math (the launch checks the sizes); the positions of a window row are
// loaded 8 at a time before they are folded in, in order, so the loads overlap.
struct PoolGeom32 {
  int32_t n, c, h, w, kh, kw, sh, sw, ph, pw, oh, ow;
};

// KWF: the window width when it is fixed at compile time (3 for the ResNet stem pool), so a row takes exactly
// that many loads; 0: any width, loaded 8 columns at a time.
template <typename T, int MODE, int VW, int KWF = 0>
__global__ __launch_bounds__(256) void pool2d_nhwc_kernel(const typename Io<T>::storage* __restrict__ x,
                                                          typename Io<T>::storage* __restrict__ y, PoolGeom32 g) {
  using S = typename Io<T>::storage;
  struct Vec {
    S v[VW];
  };
  const int groups = g.c / VW;
  const int total = g.n * g.oh * g.ow * groups;
  const int stride = gridDim.x * blockDim.x;
  const float denom = static_cast<float>(g.kh * g.kw);
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int cg = i % groups, pix = i / groups;
    const int ow = pix % g.ow, oh = (pix / g.ow) % g.oh, n = pix / (g.ow * g.oh);
    float acc[VW];
    bool found = false;
#pragma unroll
    for (int e = 0; e < VW; ++e) acc[e] = 0.0f;
    for (int a = 0; a < g.kh; ++a) {
      const int ih = oh * g.sh - g.ph + a;
      if (ih < 0 || ih >= g.h) continue;
      const S* row = x + (static_cast<int64_t>(n * g.h + ih) * g.w) * g.c + cg * VW;
      constexpr int U = KWF > 0 ? KWF : 8;
      for (int b0 = 0; b0 < g.kw; b0 += U) {
        Vec vals[U];
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int iw = ow * g.sw - g.pw + b0 + u;
          ok[u] = b0 + u < g.kw && iw >= 0 && iw < g.w;
          const int iwc = iw < 0 ? 0 : (iw >= g.w ? g.w - 1 : iw);  // clamped: the load is unconditional
          const S* src = row + static_cast<int64_t>(iwc) * g.c;
          if constexpr (VW * sizeof(S) == 16) {
            const uint4 w = *reinterpret_cast<const uint4*>(src);
            __builtin_memcpy(vals[u].v, &w, 16);
          } else {
#pragma unroll
            for (int e = 0; e < VW; ++e) vals[u].v[e] = src[e];
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (!ok[u]) continue;
#pragma unroll
          for (int e = 0; e < VW; ++e) {
            const float f = Io<T>::load(vals[u].v[e]);
            if (MODE == 0) {
              if (!found || f > acc[e]) acc[e] = f;
            } else {
              acc[e] += f;
            }
          }
          found = true;
        }
      }
    }
    S o[VW];
#pragma unroll
    for (int e = 0; e < VW; ++e) o[e] = Io<T>::store(MODE == 0 ? acc[e] : acc[e] / denom);
    S* dst = y + static_cast<int64_t>(pix) * g.c + cg * VW;
    if constexpr (VW * sizeof(S) == 16) {
      uint4 w;
      __builtin_memcpy(&w, o, 16);
      *reinterpret_cast<uint4*>(dst) = w;
    } else {
#pragma unroll
      for (int e = 0; e < VW; ++e) dst[e] = o[e];
    }
  }
}

// Pooling over whole planes (a 1 x 1 output, the window the plane, no padding; ResNet's global average pool):
// thread = (image, pair of channels). All the pair's plane positions are loaded before the first is used, then
// folded in the plane's row-major order, the order of pool2d_nhwc_kernel, so the results are the same bit for
// bit. Two channels per thread (4-byte loads, 64 lanes on 256 contiguous bytes of a pixel) give 32 x more
// threads than 16-byte vectors and one memory latency per thread.
constexpr int kGlobalPoolMax = 64;  // plane positions per thread
template <typename T, int MODE>
__global__ __launch_bounds__(256) void pool_global_nhwc_kernel(const typename Io<T>::storage* __restrict__ x,
                                                               typename Io<T>::storage* __restrict__ y, int32_t n,
                                                               int32_t c, int32_t hw) {
  using S = typename Io<T>::storage;
  constexpr int VW = sizeof(S) == 2 ? 2 : 1;
  struct Vec {
    S v[VW];
  };
  const int pairs = c / VW;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * pairs) return;
  const int img = i / pairs, cp = i - img * pairs;
  const Vec* src = reinterpret_cast<const Vec*>(x + static_cast<int64_t>(img) * hw * c) + cp;
  // every load unconditional (positions past the plane re-read its last one, never used), so none waits behind a
  // branch and all are in flight together
  Vec vals[kGlobalPoolMax];
#pragma unroll
  for (int p = 0; p < kGlobalPoolMax; ++p) vals[p] = src[static_cast<int64_t>(min(p, hw - 1)) * pairs];
  float acc[VW];
#pragma unroll
  for (int e = 0; e < VW; ++e) acc[e] = 0.0f;
#pragma unroll
  for (int p = 0; p < kGlobalPoolMax; ++p) {
    if (p >= hw) continue;  // uniform; no break, so the loop unrolls and vals keeps constant indices (registers)
#pragma unroll
    for (int e = 0; e < VW; ++e) {
      const float f = Io<T>::load(vals[p].v[e]);
      if (MODE == 0) {
        if (p == 0 || f > acc[e]) acc[e] = f;
      } else {
        acc[e] += f;
      }
    }
  }
  const float denom = static_cast<float>(hw);
  Vec o;
#pragma unroll
  for (int e = 0; e < VW; ++e) o.v[e] = Io<T>::store(MODE == 0 ? acc[e] : acc[e] / denom);
  reinterpret_cast<Vec*>(y + static_cast<int64_t>(img) * c)[cp] = o;
}

template <typename T>
fh_status launch_pool_nhwc(int32_t mode, const void* x, void* y, const PoolGeom& g, hipStream_t s) {
  using S = typename Io<T>::storage;
  constexpr int V = 16 / static_cast<int>(sizeof(S));
  const bool vec = g.c % V == 0 && aligned16(x) && aligned16(y);
  const int64_t total = g.n * g.oh * g.ow * (vec ? g.c / V : g.c);
  if (total >= (int64_t{1} << 31) || g.n * g.h * g.w >= (int64_t{1} << 31) || g.c >= (int64_t{1} << 31))
    return fail(FH_UNIMPLEMENTED, "fh_pool2d_nhwc: more than 2^31 outputs or input pixels");
  const PoolGeom32 g32{static_cast<int32_t>(g.n),  static_cast<int32_t>(g.c),  static_cast<int32_t>(g.h),
                       static_cast<int32_t>(g.w),  static_cast<int32_t>(g.kh), static_cast<int32_t>(g.kw),
                       static_cast<int32_t>(g.sh), static_cast<int32_t>(g.sw), static_cast<int32_t>(g.ph),
                       static_cast<int32_t>(g.pw), static_cast<int32_t>(g.oh), static_cast<int32_t>(g.ow)};
  if (g.oh == 1 && g.ow == 1 && g.ph == 0 && g.pw == 0 && g.kh == g.h && g.kw == g.w && g.h * g.w <= kGlobalPoolMax &&
      g.c % (sizeof(S) == 2 ? 2 : 1) == 0 && (reinterpret_cast<uintptr_t>(x) & 3) == 0 &&
      (reinterpret_cast<uintptr_t>(y) & 3) == 0) {
    const int32_t hw = static_cast<int32_t>(g.h * g.w), pairs = static_cast<int32_t>(g.c / (sizeof(S) == 2 ? 2 : 1));
    const dim3 grid(static_cast<uint32_t>((g.n * pairs + 255) / 256));
    const auto* xs = static_cast<const S*>(x);
    auto* ys = static_cast<S*>(y);
    const int32_t n32 = static_cast<int32_t>(g.n), c32 = static_cast<int32_t>(g.c);
    if (mode == 0) hipLaunchKernelGGL((pool_global_nhwc_kernel<T, 0>), grid, dim3(256), 0, s, xs, ys, n32, c32, hw);
    else hipLaunchKernelGGL((pool_global_nhwc_kernel<T, 1>), grid, dim3(256), 0, s, xs, ys, n32, c32, hw);
    return launch_status("pool_global_nhwc_kernel launch");
  }
  int64_t blocks = (total + 255) / 256;
  const int64_t cap = static_cast<int64_t>(device_cu_count()) * 16;
  if (blocks > cap) blocks = cap;
  const dim3 grid(static_cast<uint32_t>(blocks));
  const auto* xs = static_cast<const S*>(x);
  auto* ys = static_cast<S*>(y);
  if (vec && g.kw == 3) {
    if (mode == 0) hipLaunchKernelGGL((pool2d_nhwc_kernel<T, 0, V, 3>), grid, dim3(256), 0, s, xs, ys, g32);
    else hipLaunchKernelGGL((pool2d_nhwc_kernel<T, 1, V, 3>), grid, dim3(256), 0, s, xs, ys, g32);
  } else if (vec) {
    if (mode == 0) hipLaunchKernelGGL((pool2d_nhwc_kernel<T, 0, V>), grid, dim3(256), 0, s, xs, ys, g32);
    else hipLaunchKernelGGL((pool2d_nhwc_kernel<T, 1, V>), grid, dim3(256), 0, s, xs, ys, g32);
  } else {
    if (mode == 0) hipLaunchKernelGGL((pool2d_nhwc_kernel<T, 0, 1>), grid, dim3(256), 0, s, xs, ys, g32);
    else hipLaunchKernelGGL((pool2d_nhwc_kernel<T, 1, 1>), grid, dim3(256), 0, s, xs, ys, g32);
  }
  return launch_status("pool2d_nhwc_kernel launch");
}

}  // namespace
}  // namespace fh

using namespace fh;

namespace {

// Shared argument checks of the pooling entry points; fills g (with Ho, Wo) or returns the error.
fh_status check_pool(const char* who, int32_t dtype, int32_t mode, const int64_t* geom, PoolGeom& g) {
  const std::string w(who);
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, w + ": unsupported dtype");
  if (mode != 0 && mode != 1) return fail(FH_INVALID_ARGUMENT, w + ": mode must be 0 (max) or 1 (avg)");
  if (geom == nullptr) return fail(FH_INVALID_ARGUMENT, w + ": null geometry");
  g = PoolGeom{geom[0], geom[1], geom[2], geom[3], geom[4], geom[5], geom[6], geom[7], geom[8], geom[9], 0, 0};
  if (g.n < 0 || g.c < 0 || g.h < 0 || g.w < 0 || g.kh <= 0 || g.kw <= 0 || g.sh <= 0 || g.sw <= 0 || g.ph < 0 ||
      g.pw < 0)
    return fail(FH_INVALID_ARGUMENT, w + ": invalid geometry");
  if (g.h + 2 * g.ph < g.kh || g.w + 2 * g.pw < g.kw)
    return fail(FH_INVALID_ARGUMENT, w + ": window larger than the padded input");
  g.oh = (g.h + 2 * g.ph - g.kh) / g.sh + 1;
  g.ow = (g.w + 2 * g.pw - g.kw) / g.sw + 1;
  if (mode == 0) {
    // Every window must hold a valid position: the last window start must not lie beyond the input and the
    // first window must reach into it (reference rejects such windows with kInternal).
    if (g.ph >= g.kh || g.pw >= g.kw || (g.oh - 1) * g.sh - g.ph >= g.h || (g.ow - 1) * g.sw - g.pw >= g.w)
      return fail(FH_INVALID_ARGUMENT, w + ": a max-pool window has no valid (non-padding) position");
  }
  return FH_OK;
}

}  // namespace

extern "C" fh_status fh_pool2d(int32_t dtype, int32_t mode, const void* x, void* y, const int64_t geom[10],
                               void* stream) {
  PoolGeom g{};
  if (fh_status st = check_pool("fh_pool2d", dtype, mode, geom, g); st != FH_OK) return st;
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

extern "C" fh_status fh_pool2d_nhwc(int32_t dtype, int32_t mode, const void* x, void* y, const int64_t geom[10],
                                    void* stream) {
  PoolGeom g{};
  if (fh_status st = check_pool("fh_pool2d_nhwc", dtype, mode, geom, g); st != FH_OK) return st;
  if (g.n * g.c * g.oh * g.ow == 0) return FH_OK;
  if (x == nullptr || y == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_pool2d_nhwc: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case FH_F32:
      return launch_pool_nhwc<float>(mode, x, y, g, s);
    case FH_BF16:
      return launch_pool_nhwc<bf16_t>(mode, x, y, g, s);
    default:
      return launch_pool_nhwc<f16_t>(mode, x, y, g, s);
  }
}

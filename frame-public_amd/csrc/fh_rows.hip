// Row reductions over the last axis of [rows, cols]: softmax and LayerNorm.
//
// One wavefront (64 lanes) owns a row when the row fits in registers (cols <= 64 * 32): the row is read
// once, reduced with cross-lane shuffles, and written once. Longer rows fall back to one workgroup per row
// that streams the row through global memory in three passes.
//
// softmax (reference: src/backends/cpu/kernels/sequence.cpp:114-174): m = max, e = exp(x - m), s = sum(e),
// y = round(e / s). LayerNorm (reference: src/backends/cpu/kernels/sequence.cpp:182-279): two-pass mean and
// variance, r = 1 / sqrt(var + eps), y = round(gamma * ((x - mean) * r) + beta). All arithmetic in fp32;
// multiplies and adds are not contracted, division and sqrt are correctly rounded. For 16-bit outputs the softmax
// of the register-resident kernels evaluates e as 2^((x - m) log2 e) on v_exp_f32 and y as round(e * (1 / s)): the
// same d = x - m as the reference, an exponential within a few fp32 ulps of expf and a quotient within one, which
// changes a stored 8- or 11-bit probability only where it lies that close to a rounding boundary. expf and the
// correctly rounded division cost about 25 VALU instructions per element and made the [65536, 512] bf16 softmax
// instruction-bound (30.7 us for 134 MB); fp32 outputs keep them.
#include <hip/hip_runtime.h>

#include <string>
#include <type_traits>

#include "fh_common.h"

namespace fh {
namespace {

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float other = __shfl_xor(v, o, 64);
    v = (other > v) ? other : v;
  }
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

constexpr int kRowsPerBlock = 4;  // 4 waves, one row each

// softmax's e = exp(d) for d = x - m: expf for fp32 outputs, 2^(d log2 e) on v_exp_f32 for 16-bit ones
template <typename T>
__device__ __forceinline__ float softmax_exp(float d) {
  if constexpr (std::is_same_v<T, float>) {
    return expf(d);
  } else {
    return __builtin_amdgcn_exp2f(d * 1.44269504088896340736f);
  }
}
// y = e / s: correctly rounded for fp32 outputs, e * (1 / s) (r passed in) for 16-bit ones
template <typename T>
__device__ __forceinline__ float softmax_div(float e, float s, float r) {
  if constexpr (std::is_same_v<T, float>) {
    return e / s;
  } else {
    return e * r;
  }
}

typedef unsigned int u4_t __attribute__((ext_vector_type(4)));

template <typename T, int PER>
__global__ __launch_bounds__(256) void softmax_wave_kernel(const typename Io<T>::storage* __restrict__ x,
                                                           typename Io<T>::storage* __restrict__ y, int64_t rows,
                                                           int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const auto* xr = x + row * cols;
  auto* yr = y + row * cols;
  float v[PER];
  float m = -__builtin_inff();
#pragma unroll
  for (int t = 0; t < PER; ++t) {
    const int64_t j = lane + 64 * t;
    v[t] = (j < cols) ? Io<T>::load(xr[j]) : -__builtin_inff();
    m = (v[t] > m) ? v[t] : m;
  }
  m = wave_max(m);
  float s = 0.0f;
#pragma unroll
  for (int t = 0; t < PER; ++t) {
    const int64_t j = lane + 64 * t;
    v[t] = (j < cols) ? softmax_exp<T>(v[t] - m) : 0.0f;
    s += v[t];
  }
  s = wave_sum(s);
  const float r = 1.0f / s;
#pragma unroll
  for (int t = 0; t < PER; ++t) {
    const int64_t j = lane + 64 * t;
    if (j < cols) yr[j] = Io<T>::store(softmax_div<T>(v[t], s, r));
  }
}

// Rows of 64 * PER elements with 16-byte aligned rows, one wave per row: lane l owns the contiguous elements
// [V*l + 64*V*t, +V) for t < PER / V, all loaded (16-byte accesses) before the max reduction. The arithmetic is
// softmax_wave_kernel's (m = max, e = exp(x - m), s = sum e, y = round(e / s)); only the order of the terms of
// the lane's partial sum differs.
template <typename T, int PER>
__global__ __launch_bounds__(256) void softmax_vec_kernel(const typename Io<T>::storage* __restrict__ x,
                                                         typename Io<T>::storage* __restrict__ y, int64_t rows) {
  using S = typename Io<T>::storage;
  constexpr int V = 16 / static_cast<int>(sizeof(S));
  constexpr int NV = PER / V;
  constexpr int64_t COLS = 64 * PER;
  static_assert(PER % V == 0, "whole vectors per lane");
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const u4_t* xr = reinterpret_cast<const u4_t*>(x + row * COLS);
  u4_t* yr = reinterpret_cast<u4_t*>(y + row * COLS);
  u4_t xv[NV];
#pragma unroll
  for (int t = 0; t < NV; ++t) xv[t] = __builtin_nontemporal_load(xr + lane + 64 * t);
  float v[PER];
  float m = -__builtin_inff();
#pragma unroll
  for (int t = 0; t < NV; ++t) {
    S e[V];
    __builtin_memcpy(e, &xv[t], 16);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      v[t * V + i] = Io<T>::load(e[i]);
      m = (v[t * V + i] > m) ? v[t * V + i] : m;
    }
  }
  m = wave_max(m);
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    v[i] = softmax_exp<T>(v[i] - m);
    s += v[i];
  }
  s = wave_sum(s);
  const float r = 1.0f / s;
#pragma unroll
  for (int t = 0; t < NV; ++t) {
    S o[V];
#pragma unroll
    for (int i = 0; i < V; ++i) o[i] = Io<T>::store(softmax_div<T>(v[t * V + i], s, r));
    u4_t w;
    __builtin_memcpy(&w, o, 16);
    __builtin_nontemporal_store(w, yr + lane + 64 * t);
  }
}

__device__ float block_reduce(float v, bool is_max, float* scratch) {
  v = is_max ? wave_max(v) : wave_sum(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) scratch[w] = v;
  __syncthreads();
  float r = scratch[0];
  for (int k = 1; k < static_cast<int>(blockDim.x >> 6); ++k)
    r = is_max ? ((scratch[k] > r) ? scratch[k] : r) : r + scratch[k];
  __syncthreads();
  return r;
}

template <typename T>
__global__ __launch_bounds__(256) void softmax_block_kernel(const typename Io<T>::storage* __restrict__ x,
                                                            typename Io<T>::storage* __restrict__ y, int64_t cols) {
  __shared__ float scratch[4];
  const auto* xr = x + static_cast<int64_t>(blockIdx.x) * cols;
  auto* yr = y + static_cast<int64_t>(blockIdx.x) * cols;
  float m = -__builtin_inff();
  for (int64_t j = threadIdx.x; j < cols; j += blockDim.x) {
    const float v = Io<T>::load(xr[j]);
    m = (v > m) ? v : m;
  }
  m = block_reduce(m, true, scratch);
  float s = 0.0f;
  for (int64_t j = threadIdx.x; j < cols; j += blockDim.x) s += expf(Io<T>::load(xr[j]) - m);
  s = block_reduce(s, false, scratch);
  for (int64_t j = threadIdx.x; j < cols; j += blockDim.x) yr[j] = Io<T>::store(expf(Io<T>::load(xr[j]) - m) / s);
}

template <typename T, int PER>
__global__ __launch_bounds__(256) void layer_norm_wave_kernel(const typename Io<T>::storage* __restrict__ x,
                                                              const typename Io<T>::storage* __restrict__ gamma,
                                                              const typename Io<T>::storage* __restrict__ beta,
                                                              typename Io<T>::storage* __restrict__ y,
                                                              int64_t rows, int64_t cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const auto* xr = x + row * cols;
  auto* yr = y + row * cols;
  float v[PER];
  float sum = 0.0f;
#pragma unroll
  for (int t = 0; t < PER; ++t) {
    const int64_t j = lane + 64 * t;
    v[t] = (j < cols) ? Io<T>::load(xr[j]) : 0.0f;
    sum += v[t];
  }
  const float mean = wave_sum(sum) / static_cast<float>(cols);
  float var_sum = 0.0f;
#pragma unroll
  for (int t = 0; t < PER; ++t) {
    const int64_t j = lane + 64 * t;
    const float c = v[t] - mean;
    var_sum += (j < cols) ? c * c : 0.0f;
  }
  const float variance = wave_sum(var_sum) / static_cast<float>(cols);
  const float r = 1.0f / sqrtf(variance + eps);
#pragma unroll
  for (int t = 0; t < PER; ++t) {
    const int64_t j = lane + 64 * t;
    if (j < cols) {
      const float xhat = (v[t] - mean) * r;
      const float g = Io<T>::load(gamma[j]);
      const float b = Io<T>::load(beta[j]);
      yr[j] = Io<T>::store(g * xhat + b);
    }
  }
}

// Same arithmetic with 16-byte accesses, for rows of exactly 64 * PER elements (PER a multiple of the vector
// width): lane l owns the contiguous elements [V*l + 64*V*t, +V) for t < PER / V. Every load (x, gamma, beta)
// is issued before the first reduction, so one memory latency covers the row.
template <typename T, int PER>
__global__ __launch_bounds__(256) void layer_norm_vec_kernel(const typename Io<T>::storage* __restrict__ x,
                                                             const typename Io<T>::storage* __restrict__ gamma,
                                                             const typename Io<T>::storage* __restrict__ beta,
                                                             typename Io<T>::storage* __restrict__ y, int64_t rows,
                                                             float eps) {
  using S = typename Io<T>::storage;
  constexpr int V = 16 / static_cast<int>(sizeof(S));
  constexpr int NV = PER / V;
  constexpr int64_t COLS = 64 * PER;
  static_assert(PER % V == 0, "whole vectors per lane");
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const u4_t* xr = reinterpret_cast<const u4_t*>(x + row * COLS);
  const u4_t* gr = reinterpret_cast<const u4_t*>(gamma);
  const u4_t* br = reinterpret_cast<const u4_t*>(beta);
  u4_t* yr = reinterpret_cast<u4_t*>(y + row * COLS);
  u4_t xv[NV], gv[NV], bv[NV];
#pragma unroll
  for (int t = 0; t < NV; ++t) xv[t] = __builtin_nontemporal_load(xr + lane + 64 * t);
#pragma unroll
  for (int t = 0; t < NV; ++t) {
    gv[t] = gr[lane + 64 * t];
    bv[t] = br[lane + 64 * t];
  }
  float v[PER];
  float sum = 0.0f;
#pragma unroll
  for (int t = 0; t < NV; ++t) {
    S e[V];
    __builtin_memcpy(e, &xv[t], 16);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      v[t * V + i] = Io<T>::load(e[i]);
      sum += v[t * V + i];
    }
  }
  const float mean = wave_sum(sum) / static_cast<float>(COLS);
  float var_sum = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    v[i] -= mean;  // x - mean, kept for the normalisation (the same fp32 value the reference computes twice)
    var_sum += v[i] * v[i];
  }
  const float variance = wave_sum(var_sum) / static_cast<float>(COLS);
  const float r = 1.0f / sqrtf(variance + eps);
#pragma unroll
  for (int t = 0; t < NV; ++t) {
    S g[V], b[V];
    __builtin_memcpy(g, &gv[t], 16);
    __builtin_memcpy(b, &bv[t], 16);
    float o[V];
#pragma unroll
    for (int i = 0; i < V; ++i) o[i] = Io<T>::load(g[i]) * (v[t * V + i] * r) + Io<T>::load(b[i]);
    const uint4 pw = pack_vec<T>(o);
    __builtin_nontemporal_store(u4_t{pw.x, pw.y, pw.z, pw.w}, yr + lane + 64 * t);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void layer_norm_block_kernel(const typename Io<T>::storage* __restrict__ x,
                                                               const typename Io<T>::storage* __restrict__ gamma,
                                                               const typename Io<T>::storage* __restrict__ beta,
                                                               typename Io<T>::storage* __restrict__ y, int64_t cols,
                                                               float eps) {
  __shared__ float scratch[4];
  const auto* xr = x + static_cast<int64_t>(blockIdx.x) * cols;
  auto* yr = y + static_cast<int64_t>(blockIdx.x) * cols;
  float sum = 0.0f;
  for (int64_t j = threadIdx.x; j < cols; j += blockDim.x) sum += Io<T>::load(xr[j]);
  const float mean = block_reduce(sum, false, scratch) / static_cast<float>(cols);
  float var_sum = 0.0f;
  for (int64_t j = threadIdx.x; j < cols; j += blockDim.x) {
    const float c = Io<T>::load(xr[j]) - mean;
    var_sum += c * c;
  }
  const float variance = block_reduce(var_sum, false, scratch) / static_cast<float>(cols);
  const float r = 1.0f / sqrtf(variance + eps);
  for (int64_t j = threadIdx.x; j < cols; j += blockDim.x) {
    const float xhat = (Io<T>::load(xr[j]) - mean) * r;
    yr[j] = Io<T>::store(Io<T>::load(gamma[j]) * xhat + Io<T>::load(beta[j]));
  }
}

template <typename T, template <typename, int> class Launcher, typename... Args>
fh_status by_width(int64_t cols, Args... args) {
  if (cols <= 64) return Launcher<T, 1>::go(args...);
  if (cols <= 128) return Launcher<T, 2>::go(args...);
  if (cols <= 256) return Launcher<T, 4>::go(args...);
  if (cols <= 512) return Launcher<T, 8>::go(args...);
  if (cols <= 1024) return Launcher<T, 16>::go(args...);
  return Launcher<T, 32>::go(args...);
}

template <typename T, int PER>
struct SoftmaxLaunch {
  using S = typename Io<T>::storage;
  static fh_status go(const void* x, void* y, int64_t rows, int64_t cols, hipStream_t s) {
    const dim3 grid(static_cast<uint32_t>((rows + kRowsPerBlock - 1) / kRowsPerBlock));
    hipLaunchKernelGGL((softmax_wave_kernel<T, PER>), grid, dim3(256), 0, s, static_cast<const S*>(x),
                       static_cast<S*>(y), rows, cols);
    return launch_status("softmax_wave_kernel launch");
  }
};

template <typename T, int PER>
struct LayerNormLaunch {
  using S = typename Io<T>::storage;
  static fh_status go(const void* x, const void* g, const void* b, void* y, int64_t rows, int64_t cols, float eps,
                      hipStream_t s) {
    const dim3 grid(static_cast<uint32_t>((rows + kRowsPerBlock - 1) / kRowsPerBlock));
    hipLaunchKernelGGL((layer_norm_wave_kernel<T, PER>), grid, dim3(256), 0, s, static_cast<const S*>(x),
                       static_cast<const S*>(g), static_cast<const S*>(b), static_cast<S*>(y), rows, cols, eps);
    return launch_status("layer_norm_wave_kernel launch");
  }
};

template <typename T, int PER>
fh_status launch_softmax_vec(const void* x, void* y, int64_t rows, hipStream_t s) {
  using S = typename Io<T>::storage;
  const dim3 grid(static_cast<uint32_t>((rows + kRowsPerBlock - 1) / kRowsPerBlock));
  hipLaunchKernelGGL((softmax_vec_kernel<T, PER>), grid, dim3(256), 0, s, static_cast<const S*>(x),
                     static_cast<S*>(y), rows);
  return launch_status("softmax_vec_kernel launch");
}

bool aligned16(const void* p);

template <typename T>
fh_status softmax_typed(const void* x, void* y, int64_t rows, int64_t cols, hipStream_t s) {
  using S = typename Io<T>::storage;
  constexpr int V = 16 / static_cast<int>(sizeof(S));
  if (aligned16(x) && aligned16(y)) {
    if (cols == 64 * V) return launch_softmax_vec<T, V>(x, y, rows, s);
    if (cols == 64 * 2 * V) return launch_softmax_vec<T, 2 * V>(x, y, rows, s);
    if (cols == 64 * 4 * V) return launch_softmax_vec<T, 4 * V>(x, y, rows, s);
  }
  if (cols <= 64 * 32) return by_width<T, SoftmaxLaunch>(cols, x, y, rows, cols, s);
  hipLaunchKernelGGL(softmax_block_kernel<T>, dim3(static_cast<uint32_t>(rows)), dim3(256), 0, s,
                     static_cast<const S*>(x), static_cast<S*>(y), cols);
  return launch_status("softmax_block_kernel launch");
}

template <typename T, int PER>
fh_status launch_layer_norm_vec(const void* x, const void* g, const void* b, void* y, int64_t rows, float eps,
                                hipStream_t s) {
  using S = typename Io<T>::storage;
  const dim3 grid(static_cast<uint32_t>((rows + kRowsPerBlock - 1) / kRowsPerBlock));
  hipLaunchKernelGGL((layer_norm_vec_kernel<T, PER>), grid, dim3(256), 0, s, static_cast<const S*>(x),
                     static_cast<const S*>(g), static_cast<const S*>(b), static_cast<S*>(y), rows, eps);
  return launch_status("layer_norm_vec_kernel launch");
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <typename T>
fh_status layer_norm_typed(const void* x, const void* g, const void* b, void* y, int64_t rows, int64_t cols,
                           float eps, hipStream_t s) {
  using S = typename Io<T>::storage;
  if (aligned16(x) && aligned16(g) && aligned16(b) && aligned16(y)) {
    constexpr int V = 16 / static_cast<int>(sizeof(S));
    if (cols == 64 * V) return launch_layer_norm_vec<T, V>(x, g, b, y, rows, eps, s);
    if (cols == 64 * 2 * V) return launch_layer_norm_vec<T, 2 * V>(x, g, b, y, rows, eps, s);
    if (cols == 64 * 4 * V) return launch_layer_norm_vec<T, 4 * V>(x, g, b, y, rows, eps, s);
    if (V == 4 && cols == 64 * 8 * V) return launch_layer_norm_vec<T, 8 * V>(x, g, b, y, rows, eps, s);
  }
  if (cols <= 64 * 32) return by_width<T, LayerNormLaunch>(cols, x, g, b, y, rows, cols, eps, s);
  hipLaunchKernelGGL(layer_norm_block_kernel<T>, dim3(static_cast<uint32_t>(rows)), dim3(256), 0, s,
                     static_cast<const S*>(x), static_cast<const S*>(g), static_cast<const S*>(b), static_cast<S*>(y),
                     cols, eps);
  return launch_status("layer_norm_block_kernel launch");
}

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" fh_status fh_softmax_rows(int32_t dtype, const void* x, void* y, int64_t rows, int64_t cols,
                                     void* stream) {
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, "fh_softmax_rows: unsupported dtype");
  if (rows < 0 || cols < 0) return fail(FH_INVALID_ARGUMENT, "fh_softmax_rows: negative size");
  if (rows == 0 || cols == 0) return FH_OK;
  if (rows > 0x7fffffffLL) return fail(FH_INVALID_ARGUMENT, "fh_softmax_rows: too many rows");
  if (x == nullptr || y == nullptr) return fail(FH_INVALID_ARGUMENT, "fh_softmax_rows: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case FH_F32:
      return softmax_typed<float>(x, y, rows, cols, s);
    case FH_BF16:
      return softmax_typed<bf16_t>(x, y, rows, cols, s);
    default:
      return softmax_typed<f16_t>(x, y, rows, cols, s);
  }
}

extern "C" fh_status fh_layer_norm_rows(int32_t dtype, const void* x, const void* gamma, const void* beta, void* y,
                                        int64_t rows, int64_t cols, float eps, void* stream) {
  if (!is_supported_float(dtype)) return fail(FH_UNIMPLEMENTED, "fh_layer_norm_rows: unsupported dtype");
  if (rows < 0 || cols < 0) return fail(FH_INVALID_ARGUMENT, "fh_layer_norm_rows: negative size");
  if (rows == 0 || cols == 0) return FH_OK;
  if (rows > 0x7fffffffLL) return fail(FH_INVALID_ARGUMENT, "fh_layer_norm_rows: too many rows");
  if (x == nullptr || gamma == nullptr || beta == nullptr || y == nullptr)
    return fail(FH_INVALID_ARGUMENT, "fh_layer_norm_rows: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case FH_F32:
      return layer_norm_typed<float>(x, gamma, beta, y, rows, cols, eps, s);
    case FH_BF16:
      return layer_norm_typed<bf16_t>(x, gamma, beta, y, rows, cols, eps, s);
    default:
      return layer_norm_typed<f16_t>(x, gamma, beta, y, rows, cols, eps, s);
  }
}

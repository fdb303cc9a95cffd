// Shared helpers of the gfx950 kernel library: error plumbing for the C ABI and the exact
// fp32 <-> 16-bit conversions every kernel uses for loads and stores.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <string>

#include "frame_hip_abi.h"

namespace fh {

// Thread-local message behind fh_last_error().
void set_error(const std::string& message);
fh_status fail(fh_status code, const std::string& message);
fh_status check_hip(hipError_t err, const char* what);

#define FH_HIP_CHECK(expr)                                      \
  do {                                                          \
    hipError_t fh_err_ = (expr);                                \
    if (fh_err_ != hipSuccess) return ::fh::check_hip(fh_err_, #expr); \
  } while (0)

// Checks the launch status of the most recent kernel launch on this thread.
inline fh_status launch_status(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return check_hip(err, what);
  return FH_OK;
}

inline bool is_supported_float(int32_t dtype) {
  return dtype == FH_F32 || dtype == FH_F16 || dtype == FH_BF16;
}

inline int64_t dtype_size(int32_t dtype) { return dtype == FH_F32 ? 4 : 2; }

// ----------------------------------------------------------------------------------------------
// Storage types and conversions. 16-bit values travel as raw uint16_t bit patterns so that the
// rounding is exactly the reference's: round-to-nearest-even, NaN forced quiet with the sign kept
// (reference: include/frame/core/dtype.h:51-131).
// ----------------------------------------------------------------------------------------------
struct bf16_t {
  uint16_t bits;
};
struct f16_t {
  uint16_t bits;
};

__host__ __device__ inline float bf16_bits_to_float(uint16_t b) {
  uint32_t u = static_cast<uint32_t>(b) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

__host__ __device__ inline uint16_t float_to_bf16_bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ inline float f16_bits_to_float(uint16_t b) {
  _Float16 h;
  __builtin_memcpy(&h, &b, 2);
  return static_cast<float>(h);  // exact widening
}

__device__ inline uint16_t float_to_f16_bits(float f) {
  if (f != f) {  // NaN: quiet NaN with the sign kept, as the reference's narrowing does
    uint32_t u;
    __builtin_memcpy(&u, &f, 4);
    return static_cast<uint16_t>(((u >> 16) & 0x8000u) | 0x7e00u);
  }
  _Float16 h = static_cast<_Float16>(f);  // v_cvt_f16_f32: IEEE round-to-nearest-even
  uint16_t b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

template <typename T>
struct Io;

template <>
struct Io<float> {
  using storage = float;
  __device__ static float load(float v) { return v; }
  __device__ static float store(float v) { return v; }
  // round-trip through storage precision (identity for fp32)
  __device__ static float round(float v) { return v; }
};

// Device narrowing to bf16 on gfx950's v_cvt_pk_bf16_f32 (round-to-nearest-even). Checked exhaustively on an
// MI355X against float_to_bf16_bits above for all 2^32 float bit patterns, NaNs and denormals included: zero
// differences, so it is the reference's narrowing.
__device__ inline uint16_t float_to_bf16_bits_hw(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

template <>
struct Io<bf16_t> {
  using storage = uint16_t;
  __device__ static float load(uint16_t v) { return bf16_bits_to_float(v); }
  __device__ static uint16_t store(float v) { return float_to_bf16_bits_hw(v); }
  __device__ static float round(float v) { return bf16_bits_to_float(float_to_bf16_bits_hw(v)); }
};

template <>
struct Io<f16_t> {
  using storage = uint16_t;
  __device__ static float load(uint16_t v) { return f16_bits_to_float(v); }
  __device__ static uint16_t store(float v) { return float_to_f16_bits(v); }
  __device__ static float round(float v) { return f16_bits_to_float(float_to_f16_bits(v)); }
};

// Elementwise sub-op semantics, all in fp32 (reference: src/backends/cpu/kernels/elementwise.cpp:146-331).
// relu keeps NaN and -0.0 exactly like std::max(x, 0.0f): returns x unless x < 0.
__device__ inline float ew_unary(uint8_t op, float x) {
  switch (op) {
    case FH_EW_RELU:
      return (x < 0.0f) ? 0.0f : x;
    case FH_EW_SQUARE:
      return x * x;
    case FH_EW_GELU:
      return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f));
    default:
      return x;
  }
}

__device__ inline float ew_binary(uint8_t op, float a, float b) {
  return op == FH_EW_MUL ? a * b : a + b;
}

__host__ __device__ inline bool ew_is_binary(uint8_t op) { return op == FH_EW_ADD || op == FH_EW_MUL; }

inline int device_cu_count() {
  static int cached = 0;
  if (cached == 0) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess) cached = prop.multiProcessorCount;
    if (cached <= 0) cached = 256;
  }
  return cached;
}

}  // namespace fh

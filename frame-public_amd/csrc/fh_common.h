// Shared helpers of the gfx950 kernel library: error plumbing for the C ABI and the exact
// fp32 <-> 16-bit conversions every kernel uses for loads and stores.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <type_traits>

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

// Two values narrowed to T's 16-bit storage and packed in one word, lo in bits 0-15. bf16 takes one
// v_cvt_pk_bf16_f32 for the pair (the narrowing of Io<bf16_t>::store); f16 narrows each half.
template <typename T>
__device__ __forceinline__ uint32_t store2(float lo, float hi) {
  if constexpr (std::is_same_v<T, bf16_t>) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{lo, hi}, b2));
  } else {
    return static_cast<uint32_t>(Io<T>::store(lo)) | (static_cast<uint32_t>(Io<T>::store(hi)) << 16);
  }
}
template <typename T>
__device__ __forceinline__ float load_lo(uint32_t w) { return Io<T>::load(static_cast<uint16_t>(w & 0xffffu)); }
template <typename T>
__device__ __forceinline__ float load_hi(uint32_t w) { return Io<T>::load(static_cast<uint16_t>(w >> 16)); }
// a, b <- round(a), round(b) through T's storage (Io<T>::round on each; identity for fp32)
template <typename T>
__device__ __forceinline__ void round_pair(float& a, float& b) {
  if constexpr (!std::is_same_v<T, float>) {
    const uint32_t w = store2<T>(a, b);
    a = load_lo<T>(w);
    b = load_hi<T>(w);
  }
}

// One 16-byte vector of T's storage <-> 16 / sizeof(storage) floats; the narrowing goes pairwise through store2.
template <typename T, int V>
__device__ __forceinline__ void unpack_vec(const uint4& w, float (&v)[V]) {
  static_assert(V * sizeof(typename Io<T>::storage) == 16, "one 16-byte vector");
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    if constexpr (std::is_same_v<T, float>) {
      v[d] = __uint_as_float(u[d]);
    } else {
      v[2 * d] = load_lo<T>(u[d]);
      v[2 * d + 1] = load_hi<T>(u[d]);
    }
  }
}
template <typename T, int V>
__device__ __forceinline__ uint4 pack_vec(const float (&v)[V]) {
  static_assert(V * sizeof(typename Io<T>::storage) == 16, "one 16-byte vector");
  uint32_t u[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    if constexpr (std::is_same_v<T, float>) {
      u[d] = __float_as_uint(v[d]);
    } else {
      u[d] = store2<T>(v[2 * d], v[2 * d + 1]);
    }
  }
  return uint4{u[0], u[1], u[2], u[3]};
}
template <typename T, int V>
__device__ __forceinline__ void round_vec(float (&v)[V]) {
#pragma unroll
  for (int x = 0; x + 1 < V; x += 2) round_pair<T>(v[x], v[x + 1]);
}

// gelu(x) = 0.5 x (1 + erf(x / sqrt 2)), with 1 + erf(z) = 2 - erfc(|z|) for x >= 0 and erfc(|z|) for x < 0, and
// erfc from the Chebyshev fit of Numerical Recipes in C (2nd ed., section 6.2, erfcc; fractional error below
// 1.2e-7 for all z): erfc(z) = t exp(-z^2 + P(t)), t = 1 / (1 + z / 2). In fp32 the result is within 1e-6
// relative of the exact function for |x| < 5 (7e-6 at x = -10, where exp(-z^2) itself limits), and it keeps
// relative accuracy in the negative tail, where 1 + erff(z) cancels to zero. About 20 instructions, no branch.
// erfc(|x| / sqrt 2) by the Numerical Recipes erfcc fit (see above).
__device__ inline float erfc_scaled_abs(float x) {
  const float z = __builtin_fabsf(x) * 0.70710678118654752440f;
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.5f, z, 1.0f));
  float p = 0.17087277f;
  p = __builtin_fmaf(p, t, -0.82215223f);
  p = __builtin_fmaf(p, t, 1.48851587f);
  p = __builtin_fmaf(p, t, -1.13520398f);
  p = __builtin_fmaf(p, t, 0.27886807f);
  p = __builtin_fmaf(p, t, -0.18628806f);
  p = __builtin_fmaf(p, t, 0.09678418f);
  p = __builtin_fmaf(p, t, 0.37409196f);
  p = __builtin_fmaf(p, t, 1.00002368f);
  p = __builtin_fmaf(p, t, -1.26551223f);
  return t * __expf(__builtin_fmaf(-z, z, p));
}

__device__ inline float gelu_erfc(float x) {
  const float erfc_z = erfc_scaled_abs(x);
  return 0.5f * x * (x >= 0.0f ? 2.0f - erfc_z : erfc_z);
}

// Elementwise sub-op semantics, all in fp32 (reference: src/backends/cpu/kernels/elementwise.cpp:146-331).
// relu keeps NaN and -0.0 exactly like std::max(x, 0.0f): returns x unless x < 0.
// The ops a GEMM / conv epilogue program may hold (epilogue_op_ok); kept apart from the rest so the contraction
// kernels' epilogues do not carry the code of the other ops.
__device__ inline float epi_unary(uint8_t op, float x) {
  switch (op) {
    case FH_EW_RELU:
      return (x < 0.0f) ? 0.0f : x;
    case FH_EW_SQUARE:
      return x * x;
    case FH_EW_GELU:
      return gelu_erfc(x);
    default:
      return x;
  }
}
__device__ inline float epi_binary(uint8_t op, float a, float b) { return op == FH_EW_MUL ? a * b : a + b; }

__device__ inline float ew_unary(uint8_t op, float x) {
  switch (op) {
    case FH_EW_RELU:
      return (x < 0.0f) ? 0.0f : x;
    case FH_EW_SQUARE:
      return x * x;
    case FH_EW_GELU:
      return gelu_erfc(x);
    case FH_EW_SIGMOID:
      if (x >= 0.0f) return 1.0f / (1.0f + __expf(-x));
      return __expf(x) / (1.0f + __expf(x));
    case FH_EW_TANH:
      return tanhf(x);
    case FH_EW_RSQRT:
      return 1.0f / sqrtf(x);  // both correctly rounded: the reference's 1.0f / std::sqrt(x)
    default:
      return x;
  }
}

// d/dx gelu(x) = Phi(x) + x phi(x), Phi from the same erfc fit as gelu_erfc (1 + erf(z) = 2 - erfc(|z|) or
// erfc(|z|)), phi(x) = exp(-x^2/2) / sqrt(2 pi).
__device__ inline float gelu_grad(float x, float gy) {
  const float erfc_z = erfc_scaled_abs(x);
  const float cdf = x >= 0.0f ? 1.0f - 0.5f * erfc_z : 0.5f * erfc_z;
  return gy * (cdf + x * (__expf(-0.5f * x * x) * 0.39894228040143267794f));
}

__device__ inline float ew_binary(uint8_t op, float a, float b) {
  if (op == FH_EW_RELU_GRAD) return a > 0.0f ? b : 0.0f;
  if (op == FH_EW_RELU_MASK) return b > 0.0f ? a : 0.0f;
  if (op == FH_EW_GELU_GRAD) return gelu_grad(a, b);
  return op == FH_EW_MUL ? a * b : a + b;
}

// Ops a GEMM / conv epilogue program may hold: add, mul, relu, square, gelu.
__host__ __device__ constexpr bool epilogue_op_ok(uint8_t op) { return op >= FH_EW_ADD && op <= FH_EW_GELU; }

__host__ __device__ constexpr bool ew_is_binary(uint8_t op) {
  return op == FH_EW_ADD || op == FH_EW_MUL || op == FH_EW_RELU_GRAD || op == FH_EW_GELU_GRAD || op == FH_EW_RELU_MASK;
}

// The fused elementwise program of a GEMM / conv epilogue (EpilogueArgs, ConvEpilogue: nseg, round_between,
// ops[], ins[]): segment s applies ops[s] to the running value, a binary op taking its second operand from
// ins[s] at the output's index, rounding to T after each segment when round_between is set. The op codes are
// read as one scalar word and the segments are unrolled with static indices: a runtime-indexed ops[s] / ins[s]
// would load the kernel argument from memory for every value.
template <typename EP>
__device__ __forceinline__ uint64_t epilogue_ops_word(const EP& ep) {
  static_assert(sizeof(ep.ops) == sizeof(uint64_t), "eight one-byte op codes");
  uint64_t w;
  __builtin_memcpy(&w, ep.ops, sizeof(w));
  return w;
}

template <typename T, typename EP>
__device__ __forceinline__ float epilogue_one(const EP& ep, float v, int64_t idx) {
  using S = typename Io<T>::storage;
  const uint64_t opw = epilogue_ops_word(ep);
#pragma unroll
  for (int s = 0; s < FH_MAX_SEGMENTS; ++s) {
    if (s >= ep.nseg) break;
    const uint8_t op = static_cast<uint8_t>(opw >> (8 * s));
    if (ew_is_binary(op)) {
      v = epi_binary(op, v, Io<T>::load(static_cast<const S*>(ep.ins[s])[idx]));
    } else {
      v = epi_unary(op, v);
    }
    if (ep.round_between) v = Io<T>::round(v);
  }
  return v;
}

// Same program on one 16-byte vector of consecutive outputs starting at index idx (16-byte aligned operands).
template <typename T, typename EP>
__device__ __forceinline__ uint4 epilogue_vec(const EP& ep, uint4 packed, int64_t idx) {
  using S = typename Io<T>::storage;
  constexpr int V = 16 / static_cast<int>(sizeof(S));
  S vals[V];
  __builtin_memcpy(vals, &packed, 16);
  float v[V];
#pragma unroll
  for (int x = 0; x < V; ++x) v[x] = Io<T>::load(vals[x]);
  const uint64_t opw = epilogue_ops_word(ep);
#pragma unroll
  for (int s = 0; s < FH_MAX_SEGMENTS; ++s) {
    if (s >= ep.nseg) break;
    const uint8_t op = static_cast<uint8_t>(opw >> (8 * s));
    if (ew_is_binary(op)) {
      const uint4 in = *reinterpret_cast<const uint4*>(static_cast<const S*>(ep.ins[s]) + idx);
      S iv[V];
      __builtin_memcpy(iv, &in, 16);
#pragma unroll
      for (int x = 0; x < V; ++x) v[x] = epi_binary(op, v[x], Io<T>::load(iv[x]));
    } else {
#pragma unroll
      for (int x = 0; x < V; ++x) v[x] = epi_unary(op, v[x]);
    }
    if (ep.round_between) {
#pragma unroll
      for (int x = 0; x < V; ++x) v[x] = Io<T>::round(v[x]);
    }
  }
#pragma unroll
  for (int x = 0; x < V; ++x) vals[x] = Io<T>::store(v[x]);
  __builtin_memcpy(&packed, vals, 16);
  return packed;
}

// Epilogue programs with kernels of their own. A GEMM / conv kernel carries its epilogue as a template parameter E:
// the fixed programs below compile to a few instructions, while kEpiAny inlines the general interpreter
// (epilogue_vec / epilogue_one: every op of every segment), several thousand instructions that the whole
// workgroup fetches when it reaches the epilogue (measured on the resident-patch C3 conv: 30.7 us with the
// interpreter in the kernel, 17.8 us without, the same arithmetic executed). Semantics are identical: the same
// epi_unary / epi_binary, rounding after every segment when round_between is set.
enum EpiKind : int {
  kEpiNone = 0,     // no program
  kEpiRelu = 1,     // relu
  kEpiAddRelu = 2,  // add(., ins[0]); relu            (ResNet residual)
  kEpiAdd = 3,      // add(., ins[0])                   (bias of [rows, cols])
  kEpiAddGelu = 4,  // add(., ins[0]); gelu            (transformer FFN up-projection)
  kEpiAddAdd = 5,   // add(., ins[0]); add(., ins[1])  (FFN down-projection + bias + residual)
  kEpiAny = 7,      // the general interpreter
};

template <int E>
struct EpiProgram {
  static constexpr int n = E == kEpiNone ? 0 : (E == kEpiRelu || E == kEpiAdd) ? 1 : 2;
  static constexpr uint8_t op0 = E == kEpiRelu ? FH_EW_RELU : FH_EW_ADD;
  static constexpr uint8_t op1 = E == kEpiAddRelu ? FH_EW_RELU : E == kEpiAddGelu ? FH_EW_GELU : FH_EW_ADD;
};

// The fixed program an epilogue holds, or kEpiAny (host side; nseg and ops as fh_epilogue / EpilogueArgs).
template <typename EP>
inline int epi_kind(const EP& ep) {
  if (ep.nseg == 0) return kEpiNone;
  if (ep.nseg == 1 && ep.ops[0] == FH_EW_RELU) return kEpiRelu;
  if (ep.nseg == 1 && ep.ops[0] == FH_EW_ADD) return kEpiAdd;
  if (ep.nseg == 2 && ep.ops[0] == FH_EW_ADD) {
    if (ep.ops[1] == FH_EW_RELU) return kEpiAddRelu;
    if (ep.ops[1] == FH_EW_GELU) return kEpiAddGelu;
    if (ep.ops[1] == FH_EW_ADD) return kEpiAddAdd;
  }
  return kEpiAny;
}

template <int E, typename T, typename EP>
__device__ __forceinline__ float epi_one(const EP& ep, float v, int64_t idx) {
  using S = typename Io<T>::storage;
  if constexpr (E == kEpiNone) {
    return v;
  } else if constexpr (E == kEpiAny) {
    return ep.nseg > 0 ? epilogue_one<T>(ep, v, idx) : v;
  } else {
    using P = EpiProgram<E>;
    const uint8_t ops[2] = {P::op0, P::op1};
#pragma unroll
    for (int s = 0; s < P::n; ++s) {
      v = ew_is_binary(ops[s]) ? epi_binary(ops[s], v, Io<T>::load(static_cast<const S*>(ep.ins[s])[idx]))
                               : epi_unary(ops[s], v);
      if (ep.round_between) v = Io<T>::round(v);
    }
    return v;
  }
}

// The value an epilogue stages for output x (the fp32 sum plus bias): rounded to the storage type and, for the
// relu-only program, already through relu. relu of a rounded value is itself a storage value and rounds to itself,
// so applying it here equals applying it after the staging round trip; the readback then runs
// epi_after_stage<E>() instead of E (no program for relu), which saves an unpack, compare and repack per element.
//
// relu(round(x)) is computed as round(x < -lim ? 0 : x), lim = half of T's smallest denormal (2^-134 for bf16,
// 2^-25 for f16, 0 for fp32): round(x) < 0 exactly when x < -lim (x in [-lim, 0) rounds to -0.0, the tie at -lim
// to even, and relu keeps -0.0), and NaN compares false and rounds to NaN as relu keeps it.
template <typename T>
__device__ __forceinline__ float relu_before_round(float x) {
  constexpr float lim = std::is_same_v<T, bf16_t> ? 0x1p-134f : std::is_same_v<T, f16_t> ? 0x1p-25f : 0.0f;
  return x < -lim ? 0.0f : x;
}
template <int E, typename T>
__device__ __forceinline__ typename Io<T>::storage epi_stage(float x) {
  if constexpr (E == kEpiRelu) {
    return Io<T>::store(relu_before_round<T>(x));
  } else {
    return Io<T>::store(x);
  }
}
// Two adjacent staged values packed in one word (16-bit storage), one narrowing for the pair on bf16.
template <int E, typename T>
__device__ __forceinline__ uint32_t epi_stage2(float x0, float x1) {
  if constexpr (E == kEpiRelu) {
    return store2<T>(relu_before_round<T>(x0), relu_before_round<T>(x1));
  } else {
    return store2<T>(x0, x1);
  }
}
template <int E>
__host__ __device__ constexpr int epi_after_stage() {
  return E == kEpiRelu ? kEpiNone : E;
}

// Split form of epi_vec for the fixed programs, so a caller can issue the operand loads of several output vectors
// before using any of them (one memory latency per batch instead of one per vector): epi_operands<E>() 16-byte
// operand vectors per output vector, epi_load fetches them, epi_apply runs the program on them. kEpiAny reads its
// own operands (epi_operands = 0; use epi_vec).
template <int E>
__host__ __device__ constexpr int epi_operands() {
  return (E == kEpiAddRelu || E == kEpiAdd || E == kEpiAddGelu) ? 1 : E == kEpiAddAdd ? 2 : 0;
}

template <int E, typename T, typename EP>
__device__ __forceinline__ void epi_load(const EP& ep, int64_t idx, uint4* in) {
  using S = typename Io<T>::storage;
#pragma unroll
  for (int s = 0; s < epi_operands<E>(); ++s) in[s] = *reinterpret_cast<const uint4*>(static_cast<const S*>(ep.ins[s]) + idx);
}

template <int E, typename T, typename EP>
__device__ __forceinline__ uint4 epi_apply(const EP& ep, uint4 packed, const uint4* in) {
  static_assert(E != kEpiAny, "the interpreter reads its own operands");
  if constexpr (E == kEpiNone) {
    return packed;
  } else {
    using P = EpiProgram<E>;
    constexpr int V = 16 / static_cast<int>(sizeof(typename Io<T>::storage));
    const uint8_t ops[2] = {P::op0, P::op1};
    float v[V];
    unpack_vec<T>(packed, v);
    int next = 0;
#pragma unroll
    for (int s = 0; s < P::n; ++s) {
      if (ew_is_binary(ops[s])) {
        float iv[V];
        unpack_vec<T>(in[next++], iv);
#pragma unroll
        for (int x = 0; x < V; ++x) v[x] = epi_binary(ops[s], v[x], iv[x]);
      } else {
#pragma unroll
        for (int x = 0; x < V; ++x) v[x] = epi_unary(ops[s], v[x]);
      }
      if (ep.round_between) round_vec<T>(v);
    }
    return pack_vec<T>(v);
  }
}

template <int E, typename T, typename EP>
__device__ __forceinline__ uint4 epi_vec(const EP& ep, uint4 packed, int64_t idx) {
  if constexpr (E == kEpiNone) {
    return packed;
  } else if constexpr (E == kEpiAny) {
    return ep.nseg > 0 ? epilogue_vec<T>(ep, packed, idx) : packed;
  } else {
    uint4 in[epi_operands<E>() > 0 ? epi_operands<E>() : 1];
    epi_load<E, T>(ep, idx, in);
    return epi_apply<E, T>(ep, packed, in);
  }
}

// CUs of the device current at the first call (256, MI355X's count, when no device is visible), read once per
// process under the function-local static's thread-safe initialisation. Launch shapes and the band conv's
// geometry choice depend on it, so the lowering (and the lowered text) of a graph does too.
inline int device_cu_count() {
  static const int cached = [] {
    int dev = 0, cus = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess) cus = prop.multiProcessorCount;
    return cus > 0 ? cus : 256;
  }();
  return cached;
}

}  // namespace fh

#pragma once
// Data types. The C++ type <-> dtype mapping is a compile-time table; dispatch_dtype() is the single place
// where a run-time dtype code turns back into a static type. Enumerator order, trait names and the
// dispatch_dtype contract match the reference (include/frame/core/dtype.h:17-318) so backend code written
// against Frame compiles unchanged.
//
// Narrowing float32 -> float16 / bfloat16 is IEEE-754 round-to-nearest-even. NaN handling follows the
// reference's rules: float16 collapses every NaN to sign|0x7e00; bfloat16 keeps the upper payload bits and
// forces the quiet bit. Widening is exact.

#include <bit>
#include <cstddef>
#include <cstdint>
#include <string_view>
#include <type_traits>
#include <utility>

#include <frame/core/macros.h>

namespace frame {

enum class DTypeCode : uint8_t {
  kFloat32 = 0,
  kFloat64,
  kFloat16,
  kBFloat16,
  kInt8,
  kInt16,
  kInt32,
  kInt64,
  kUInt8,
  kBool,
  kCount,
};

template <typename T>
struct dtype_traits;

// Storage-only 16-bit float types (no arithmetic operators).
struct float16_t {
  uint16_t bits;
};
struct bfloat16_t {
  uint16_t bits;
};

namespace detail {
// Round-to-nearest-even right shift of an unsigned mantissa by `shift` (1..31) bits.
constexpr uint32_t rne_shift(uint32_t mantissa, uint32_t shift) {
  const uint32_t kept = mantissa >> shift;
  const uint32_t rem = mantissa & ((1U << shift) - 1U);
  const uint32_t half = 1U << (shift - 1U);
  return kept + ((rem > half || (rem == half && (kept & 1U) != 0U)) ? 1U : 0U);
}
}  // namespace detail

// float32 -> IEEE binary16, round-to-nearest-even.
constexpr float16_t float_to_float16(float value) {
  const uint32_t u = std::bit_cast<uint32_t>(value);
  const uint16_t sign = static_cast<uint16_t>((u >> 16) & 0x8000U);
  const uint32_t exp32 = (u >> 23) & 0xffU;
  const uint32_t man32 = u & 0x7fffffU;
  if (exp32 == 0xffU) {  // inf / NaN
    return float16_t{static_cast<uint16_t>(sign | (man32 != 0U ? 0x7e00U : 0x7c00U))};
  }
  const int32_t e = static_cast<int32_t>(exp32) - 127;  // unbiased exponent (float32 subnormals: tiny)
  if (e > 15) return float16_t{static_cast<uint16_t>(sign | 0x7c00U)};
  if (e >= -14) {
    // normal range of binary16: 10-bit mantissa; a carry out of the mantissa bumps the exponent naturally
    const uint32_t m = detail::rne_shift(man32 | 0x800000U, 13U);  // 11 significant bits (+ possible carry)
    const uint32_t bits = (static_cast<uint32_t>(e + 15) << 10) + (m - 0x400U);
    return float16_t{static_cast<uint16_t>(sign | (bits >= 0x7c00U ? 0x7c00U : bits))};
  }
  if (exp32 == 0U || e < -25) return float16_t{sign};  // below half of the smallest subnormal (or f32 subnormal)
  // subnormal binary16: value = m * 2^-24
  const uint32_t m = detail::rne_shift(man32 | 0x800000U, static_cast<uint32_t>(-e - 1));  // -e-1 in [14, 24]
  return float16_t{static_cast<uint16_t>(sign | m)};
}

// binary16 -> float32 (exact).
constexpr float float16_to_float(float16_t value) {
  const uint32_t h = value.bits;
  const uint32_t sign = (h & 0x8000U) << 16;
  const uint32_t e = (h >> 10) & 0x1fU;
  const uint32_t m = h & 0x3ffU;
  if (e == 0x1fU) return std::bit_cast<float>(sign | 0x7f800000U | (m << 13));
  if (e != 0U) return std::bit_cast<float>(sign | ((e + 112U) << 23) | (m << 13));
  if (m == 0U) return std::bit_cast<float>(sign);
  // subnormal: normalise the leading one into the implicit bit
  const int lz = std::countl_zero(m) - 22;  // leading zeros inside the 10-bit field, 0..9
  const uint32_t mm = (m << (lz + 1)) & 0x3ffU;
  return std::bit_cast<float>(sign | (static_cast<uint32_t>(112 - lz) << 23) | (mm << 13));
}

// float32 -> bfloat16 (upper half), round-to-nearest-even; NaN keeps its upper bits with the quiet bit set.
constexpr bfloat16_t float_to_bfloat16(float value) {
  const uint32_t u = std::bit_cast<uint32_t>(value);
  if ((u & 0x7fffffffU) > 0x7f800000U) return bfloat16_t{static_cast<uint16_t>((u >> 16) | 0x40U)};
  const uint32_t lsb = (u >> 16) & 1U;
  return bfloat16_t{static_cast<uint16_t>((u + 0x7fffU + lsb) >> 16)};
}

constexpr float bfloat16_to_float(bfloat16_t value) {
  return std::bit_cast<float>(static_cast<uint32_t>(value.bits) << 16);
}

#define FRAME_DTYPE_TRAIT(T, CODE, SIZE, NAME)           \
  template <>                                            \
  struct dtype_traits<T> {                               \
    static constexpr DTypeCode code = DTypeCode::CODE;   \
    static constexpr size_t size = SIZE;                 \
    static constexpr std::string_view name = NAME;       \
  };
FRAME_DTYPE_TRAIT(float, kFloat32, 4, "float32")
FRAME_DTYPE_TRAIT(double, kFloat64, 8, "float64")
FRAME_DTYPE_TRAIT(std::int8_t, kInt8, 1, "int8")
FRAME_DTYPE_TRAIT(std::int16_t, kInt16, 2, "int16")
FRAME_DTYPE_TRAIT(std::int32_t, kInt32, 4, "int32")
FRAME_DTYPE_TRAIT(std::int64_t, kInt64, 8, "int64")
FRAME_DTYPE_TRAIT(std::uint8_t, kUInt8, 1, "uint8")
FRAME_DTYPE_TRAIT(bool, kBool, 1, "bool")
FRAME_DTYPE_TRAIT(float16_t, kFloat16, 2, "float16")
FRAME_DTYPE_TRAIT(bfloat16_t, kBFloat16, 2, "bfloat16")
#undef FRAME_DTYPE_TRAIT

template <typename T>
concept ScalarType = requires { dtype_traits<std::remove_cv_t<T>>::code; };

// Run-time -> compile-time bridge: fn.template operator()<T>() for the static type of `code`.
template <typename Fn>
decltype(auto) dispatch_dtype(DTypeCode code, Fn&& fn) {
  switch (code) {
    case DTypeCode::kFloat32:
      return std::forward<Fn>(fn).template operator()<float>();
    case DTypeCode::kFloat64:
      return std::forward<Fn>(fn).template operator()<double>();
    case DTypeCode::kFloat16:
      return std::forward<Fn>(fn).template operator()<float16_t>();
    case DTypeCode::kBFloat16:
      return std::forward<Fn>(fn).template operator()<bfloat16_t>();
    case DTypeCode::kInt8:
      return std::forward<Fn>(fn).template operator()<std::int8_t>();
    case DTypeCode::kInt16:
      return std::forward<Fn>(fn).template operator()<std::int16_t>();
    case DTypeCode::kInt32:
      return std::forward<Fn>(fn).template operator()<std::int32_t>();
    case DTypeCode::kInt64:
      return std::forward<Fn>(fn).template operator()<std::int64_t>();
    case DTypeCode::kUInt8:
      return std::forward<Fn>(fn).template operator()<std::uint8_t>();
    case DTypeCode::kBool:
      return std::forward<Fn>(fn).template operator()<bool>();
    case DTypeCode::kCount:
      break;
  }
  FRAME_CHECK(false);
  return std::forward<Fn>(fn).template operator()<float>();
}

class DType {
 public:
  constexpr explicit DType(DTypeCode code) : code_(code) {}
  template <ScalarType T>
  static constexpr DType of() {
    return DType(dtype_traits<std::remove_cv_t<T>>::code);
  }
  constexpr DTypeCode code() const { return code_; }
  constexpr size_t itemsize() const;
  constexpr std::string_view name() const;
  constexpr bool operator==(const DType&) const = default;

 private:
  DTypeCode code_;
};

namespace detail {
struct DTypeRow {
  size_t size;
  std::string_view name;
};
constexpr DTypeRow dtype_row(DTypeCode code) {
  switch (code) {
    case DTypeCode::kFloat32: return {4, "float32"};
    case DTypeCode::kFloat64: return {8, "float64"};
    case DTypeCode::kFloat16: return {2, "float16"};
    case DTypeCode::kBFloat16: return {2, "bfloat16"};
    case DTypeCode::kInt8: return {1, "int8"};
    case DTypeCode::kInt16: return {2, "int16"};
    case DTypeCode::kInt32: return {4, "int32"};
    case DTypeCode::kInt64: return {8, "int64"};
    case DTypeCode::kUInt8: return {1, "uint8"};
    case DTypeCode::kBool: return {1, "bool"};
    case DTypeCode::kCount: break;
  }
  FRAME_CHECK(false);
  return {0, {}};
}
}  // namespace detail

constexpr size_t DType::itemsize() const { return detail::dtype_row(code_).size; }
constexpr std::string_view DType::name() const { return detail::dtype_row(code_).name; }

}  // namespace frame

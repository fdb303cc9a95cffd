#pragma once
// constant op helpers (reference: include/frame/ops/constant_utils.h): the op stores its payload as a double
// array "value" with "shape" and "dtype" attributes.

#include <cstdint>
#include <string_view>
#include <unordered_map>

#include <frame/core/macros.h>
#include <frame/core/status.h>
#include <frame/core/tensor.h>
#include <frame/ir/attribute.h>

namespace frame::ops {

inline constexpr std::string_view kConstantOpName = "constant";
inline constexpr int64_t kMaxDoubleExactInteger = 9007199254740992LL;  // 2^53

// Host tensor `out` <- attrs (value[i] narrowed double -> float -> dtype with round-to-nearest-even).
FRAME_API Status fill_tensor_from_constant_attrs(const std::unordered_map<std::string, ir::AttrValue>& attrs,
                                                 Tensor& out);
FRAME_API Status encode_tensor_to_attrs(const Tensor& in, std::unordered_map<std::string, ir::AttrValue>& attrs);
FRAME_API bool is_constant_dtype_supported(DType dtype);

}  // namespace frame::ops

#pragma once
// Node attributes: a closed set of value types (reference: include/frame/ir/attribute.h).

#include <cstddef>
#include <cstdint>
#include <string>
#include <string_view>
#include <variant>
#include <vector>

#include <frame/core/dtype.h>
#include <frame/core/macros.h>
#include <frame/core/shape.h>

namespace frame::ir {

enum class AttrType : uint8_t { kInt64, kDouble, kString, kBool, kInt64Array, kDoubleArray, kDType, kShape };

using AttrValue = std::variant<int64_t, double, std::string, bool, std::vector<int64_t>, std::vector<double>,
                               DType, Shape>;

static_assert(std::variant_size_v<AttrValue> == static_cast<std::size_t>(AttrType::kShape) + 1,
              "AttrValue alternatives and AttrType enumerators must stay in step");

FRAME_API AttrType attr_type_of(const AttrValue& value);
FRAME_API std::string_view attr_type_name(AttrType type);

}  // namespace frame::ir

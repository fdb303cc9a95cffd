#pragma once
// OpSchema: backend-independent op contract built once at registration with chained builder calls
// (reference: include/frame/ops/op_schema.h:30-170; same builder names, function-pointer types and traits).

#include <cstdint>
#include <string>
#include <string_view>
#include <unordered_map>
#include <variant>
#include <vector>

#include <frame/core/macros.h>
#include <frame/core/shape.h>
#include <frame/core/status.h>
#include <frame/ir/attribute.h>
#include <frame/ir/node.h>

namespace frame::ir {
class Graph;
}

namespace frame::ops {

enum class OpTrait : uint8_t { kElementwise, kFusable, kHasSideEffect, kCommutative };

// Read-only node view handed to shape inference and decompositions (attrs borrowed for the call).
struct NodeContext {
  std::string_view op;
  std::vector<ir::TensorType> input_types;
  const std::unordered_map<std::string, ir::AttrValue>* attrs = nullptr;
  template <typename T>
  const T* attr(std::string_view name) const {
    if (attrs == nullptr) return nullptr;
    auto it = attrs->find(std::string(name));
    return it == attrs->end() ? nullptr : std::get_if<T>(&it->second);
  }
};

using ShapeInferFn = Result<std::vector<Shape>> (*)(const NodeContext&);
using DecomposeFn = Result<ir::Graph> (*)(const NodeContext&);
using GradientFn = Result<ir::Graph> (*)(const NodeContext&);

struct OpParam {
  std::string name;
  std::string doc;
};

struct OpAttrSpec {
  std::string name;
  ir::AttrType type = ir::AttrType::kInt64;
  bool required = false;
};

class FRAME_API OpSchema {
 public:
  OpSchema& input(std::string_view name, std::string_view doc) noexcept;
  OpSchema& variadic_input(std::string_view name, std::string_view doc, int32_t min_count) noexcept;
  OpSchema& output(std::string_view name, std::string_view doc) noexcept;
  OpSchema& attr(std::string_view name, ir::AttrType type, bool required) noexcept;
  OpSchema& trait(OpTrait trait) noexcept;
  OpSchema& shape_infer(ShapeInferFn fn) noexcept;
  OpSchema& decomposition(DecomposeFn fn) noexcept;
  OpSchema& gradient(GradientFn fn) noexcept;

  std::string_view name() const { return name_; }
  const std::vector<OpParam>& inputs() const { return inputs_; }
  bool has_variadic_inputs() const { return has_variadic_input_; }
  int32_t min_input_count() const { return static_cast<int32_t>(inputs_.size()) + variadic_min_count_; }
  const std::vector<OpParam>& outputs() const { return outputs_; }
  const std::vector<OpAttrSpec>& attrs() const { return attrs_; }
  bool has_trait(OpTrait t) const { return (traits_ >> static_cast<uint8_t>(t)) & 1U; }
  ShapeInferFn shape_infer() const { return shape_infer_; }
  DecomposeFn decomposition() const { return decompose_; }
  GradientFn gradient() const { return gradient_; }

 private:
  friend class OpRegistry;
  std::string name_;
  std::vector<OpParam> inputs_;
  bool has_variadic_input_ = false;
  OpParam variadic_input_param_;
  int32_t variadic_min_count_ = 0;
  std::vector<OpParam> outputs_;
  std::vector<OpAttrSpec> attrs_;
  uint8_t traits_ = 0;
  ShapeInferFn shape_infer_ = nullptr;
  DecomposeFn decompose_ = nullptr;
  GradientFn gradient_ = nullptr;
};

}  // namespace frame::ops

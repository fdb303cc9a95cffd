#pragma once
// Value / Node / TensorType of the SSA graph IR (reference: include/frame/ir/node.h:23-100).

#include <cstdint>
#include <string>
#include <string_view>
#include <unordered_map>
#include <utility>
#include <variant>
#include <vector>

#include <frame/core/device.h>
#include <frame/core/dtype.h>
#include <frame/core/macros.h>
#include <frame/core/shape.h>
#include <frame/ir/attribute.h>

namespace frame::ir {

class Node;

enum class Layout : uint8_t { kUnknown = 0, kRowMajor };

struct TensorType {
  DType dtype{DTypeCode::kFloat32};
  Shape shape;
  Layout layout = Layout::kUnknown;
  Device device{};
};

class Value {
 public:
  Value() = default;
  const TensorType& type() const { return type_; }
  Node* producer() const { return producer_; }
  int32_t output_index() const { return output_index_; }

 private:
  friend class Node;
  friend class Graph;
  TensorType type_{};
  Node* producer_ = nullptr;
  int32_t output_index_ = 0;
};

class FRAME_API Node {
 public:
  Node() = default;
  explicit Node(std::string op) : op_(std::move(op)) {}

  std::string_view op() const { return op_; }
  const std::vector<Value*>& inputs() const { return inputs_; }
  const std::vector<Value>& outputs() const { return outputs_; }
  Value* output(int32_t index) {
    if (index < 0 || static_cast<size_t>(index) >= outputs_.size()) return nullptr;
    return &outputs_[static_cast<size_t>(index)];
  }

  void set_attr(std::string name, AttrValue value);
  const AttrValue* find_attr(std::string_view name) const;
  template <typename T>
  const T* attr(std::string_view name) const {
    const AttrValue* v = find_attr(name);
    return v == nullptr ? nullptr : std::get_if<T>(v);
  }
  // Unordered; callers needing a deterministic order sort by name.
  const std::unordered_map<std::string, AttrValue>& attrs() const { return attrs_; }

 private:
  friend class Graph;
  std::string op_;
  std::vector<Value*> inputs_;
  std::vector<Value> outputs_;
  std::unordered_map<std::string, AttrValue> attrs_;
};

}  // namespace frame::ir

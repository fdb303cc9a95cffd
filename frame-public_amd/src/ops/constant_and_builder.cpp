// constant op helpers (reference: src/ops/constant_utils.cpp) and create_node_with_inferred_types
// (reference: src/ops/graph_builder.cpp).
#include <string>
#include <type_traits>
#include <utility>
#include <variant>
#include <vector>

#include <frame/ir/graph.h>
#include <frame/ops/constant_utils.h>
#include <frame/ops/graph_builder.h>
#include <frame/ops/op_registry.h>

namespace frame::ops {

bool is_constant_dtype_supported(DType dtype) {
  switch (dtype.code()) {
    case DTypeCode::kFloat32:
    case DTypeCode::kFloat16:
    case DTypeCode::kBFloat16:
    case DTypeCode::kInt32:
    case DTypeCode::kInt64:
      return true;
    default:
      return false;
  }
}

Status fill_tensor_from_constant_attrs(const std::unordered_map<std::string, ir::AttrValue>& attrs, Tensor& out) {
  auto get = [&](const char* k) -> const ir::AttrValue* {
    auto it = attrs.find(k);
    return it == attrs.end() ? nullptr : &it->second;
  };
  auto bad = [](const std::string& m) { return Status::make(ErrorCode::kInvalidArgument, "op 'constant' " + m); };
  const ir::AttrValue* v = get("value");
  if (v == nullptr) return bad("is missing required attribute 'value' (double array)");
  const auto* values = std::get_if<std::vector<double>>(v);
  if (values == nullptr) return bad("attribute 'value' has wrong type, expected double array");
  const ir::AttrValue* s = get("shape");
  if (s == nullptr) return bad("is missing required attribute 'shape'");
  const Shape* shape = std::get_if<Shape>(s);
  if (shape == nullptr) return bad("attribute 'shape' has wrong type, expected shape");
  const ir::AttrValue* d = get("dtype");
  if (d == nullptr) return bad("is missing required attribute 'dtype'");
  const DType* dtype = std::get_if<DType>(d);
  if (dtype == nullptr) return bad("attribute 'dtype' has wrong type, expected dtype");
  const int64_t n = shape->numel();
  if (static_cast<int64_t>(values->size()) != n)
    return bad("attribute 'value' has " + std::to_string(values->size()) + " element(s), attribute 'shape' " +
               shape->to_string() + " expects " + std::to_string(n));
  if (!is_constant_dtype_supported(*dtype))
    return bad("does not support dtype '" + std::string(dtype->name()) +
               "' (supported: float32/float16/bfloat16/int32/int64)");
  if (!(out.dtype() == *dtype))
    return bad("output dtype '" + std::string(out.dtype().name()) + "' does not match attribute 'dtype' '" +
               std::string(dtype->name()) + "'");
  if (!(out.shape() == *shape))
    return bad("output shape " + out.shape().to_string() + " does not match attribute 'shape' " + shape->to_string());
  void* raw = out.raw_data();
  for (int64_t i = 0; i < n; ++i) {
    const double x = (*values)[static_cast<size_t>(i)];
    switch (dtype->code()) {
      case DTypeCode::kFloat32: static_cast<float*>(raw)[i] = static_cast<float>(x); break;
      case DTypeCode::kFloat16: static_cast<float16_t*>(raw)[i] = float_to_float16(static_cast<float>(x)); break;
      case DTypeCode::kBFloat16: static_cast<bfloat16_t*>(raw)[i] = float_to_bfloat16(static_cast<float>(x)); break;
      case DTypeCode::kInt32: static_cast<int32_t*>(raw)[i] = static_cast<int32_t>(x); break;
      default: static_cast<int64_t*>(raw)[i] = static_cast<int64_t>(x); break;
    }
  }
  return Status::ok();
}

Status encode_tensor_to_attrs(const Tensor& in, std::unordered_map<std::string, ir::AttrValue>& attrs) {
  if (!is_constant_dtype_supported(in.dtype()))
    return Status::make(ErrorCode::kInvalidArgument, "op 'constant' encode does not support dtype '" +
                                                         std::string(in.dtype().name()) +
                                                         "' (supported: float32/float16/bfloat16/int32/int64)");
  const int64_t n = in.numel();
  std::vector<double> values(static_cast<size_t>(n));
  const void* raw = in.raw_data();
  for (int64_t i = 0; i < n; ++i) {
    double x = 0;
    switch (in.dtype().code()) {
      case DTypeCode::kFloat32: x = static_cast<const float*>(raw)[i]; break;
      case DTypeCode::kFloat16: x = float16_to_float(static_cast<const float16_t*>(raw)[i]); break;
      case DTypeCode::kBFloat16: x = bfloat16_to_float(static_cast<const bfloat16_t*>(raw)[i]); break;
      default: {
        const int64_t w = in.dtype().code() == DTypeCode::kInt32 ? static_cast<const int32_t*>(raw)[i]
                                                                  : static_cast<const int64_t*>(raw)[i];
        if (w > kMaxDoubleExactInteger || w < -kMaxDoubleExactInteger)
          return Status::make(ErrorCode::kInvalidArgument,
                              "op 'constant' encode: value " + std::to_string(w) + " at index " + std::to_string(i) +
                                  " exceeds the double-exact integer bound 2^53=" +
                                  std::to_string(kMaxDoubleExactInteger) +
                                  ", would lose precision when encoded as kDoubleArray");
        x = static_cast<double>(w);
      }
    }
    values[static_cast<size_t>(i)] = x;
  }
  attrs["value"] = ir::AttrValue{std::move(values)};
  attrs["shape"] = ir::AttrValue{in.shape()};
  attrs["dtype"] = ir::AttrValue{in.dtype()};
  return Status::ok();
}

namespace {
Result<ir::Node*> create_with_types(ir::Graph& graph, std::string_view op, std::vector<ir::Value*> inputs,
                                    const AttrMap& attrs, DType dtype, Device device) {
  const OpSchema* s = OpRegistry::instance().find(op);
  if (s == nullptr) return Status::make(ErrorCode::kNotFound, "op '" + std::string(op) + "' is not registered");
  if (s->shape_infer() == nullptr)
    return Status::make(ErrorCode::kInvalidArgument, "op '" + std::string(op) + "' has no shape_infer function");
  NodeContext ctx;
  ctx.op = op;
  for (const ir::Value* v : inputs) ctx.input_types.push_back(v->type());
  ctx.attrs = &attrs;
  Result<std::vector<Shape>> shapes = s->shape_infer()(ctx);
  if (!shapes.is_ok())
    return Status::make(shapes.status().code(),
                        std::string(shapes.status().message()) + " (while building op '" + std::string(op) + "')");
  std::vector<ir::TensorType> types;
  for (const Shape& sh : shapes.value()) types.push_back(ir::TensorType{dtype, sh, ir::Layout::kUnknown, device});
  Result<ir::Node*> n = graph.create_node(std::string(op), std::move(inputs), std::move(types));
  if (!n.is_ok()) return n.status();
  for (const auto& [k, v] : attrs) n.value()->set_attr(k, v);
  return n.value();
}
}  // namespace

Result<ir::Node*> create_node_with_inferred_types(ir::Graph& graph, std::string_view op,
                                                  std::vector<ir::Value*> inputs, const AttrMap& attrs) {
  if (inputs.empty() || inputs[0] == nullptr)
    return Status::make(ErrorCode::kInvalidArgument,
                        "create_node_with_inferred_types: op '" + std::string(op) +
                            "' needs at least one input (use the Device overload for 0-input ops)");
  const ir::TensorType t0 = inputs[0]->type();
  return create_with_types(graph, op, std::move(inputs), attrs, t0.dtype, t0.device);
}

Result<ir::Node*> create_node_with_inferred_types(ir::Graph& graph, std::string_view op, Device device,
                                                  const AttrMap& attrs) {
  auto it = attrs.find("dtype");
  const DType* d = it == attrs.end() ? nullptr : std::get_if<DType>(&it->second);
  if (d == nullptr)
    return Status::make(ErrorCode::kInvalidArgument, "create_node_with_inferred_types: 0-input op '" +
                                                         std::string(op) + "' needs a 'dtype' attribute");
  return create_with_types(graph, op, {}, attrs, *d, device);
}

}  // namespace frame::ops

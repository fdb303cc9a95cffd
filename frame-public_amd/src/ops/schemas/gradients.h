#pragma once
// Gradient micrographs of the forward ops (defined in gradients.cpp, attached to the schemas in schemas.cpp).
// Each returns a graph with inputs [x.., y.., gy..] and one output per forward input, as
// compiler::build_backward_graph expects.
#include <frame/ir/graph.h>
#include <frame/ops/op_schema.h>

namespace frame::ops::schemas {

Result<ir::Graph> add_gradient(const NodeContext& ctx);
Result<ir::Graph> mul_gradient(const NodeContext& ctx);
Result<ir::Graph> relu_gradient(const NodeContext& ctx);
Result<ir::Graph> square_gradient(const NodeContext& ctx);
Result<ir::Graph> matmul_gradient(const NodeContext& ctx);
Result<ir::Graph> conv2d_gradient(const NodeContext& ctx);
Result<ir::Graph> max_pool2d_gradient(const NodeContext& ctx);
Result<ir::Graph> avg_pool2d_gradient(const NodeContext& ctx);
Result<ir::Graph> reshape_gradient(const NodeContext& ctx);
Result<ir::Graph> softmax_gradient(const NodeContext& ctx);
Result<ir::Graph> layer_norm_gradient(const NodeContext& ctx);
Result<ir::Graph> transpose_gradient(const NodeContext& ctx);
Result<ir::Graph> concat_gradient(const NodeContext& ctx);
Result<ir::Graph> slice_gradient(const NodeContext& ctx);
Result<ir::Graph> sigmoid_gradient(const NodeContext& ctx);
Result<ir::Graph> tanh_gradient(const NodeContext& ctx);
Result<ir::Graph> rsqrt_gradient(const NodeContext& ctx);
Result<ir::Graph> gelu_gradient(const NodeContext& ctx);

}  // namespace frame::ops::schemas

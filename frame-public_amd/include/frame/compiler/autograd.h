#pragma once
// Compile-time reverse-mode differentiation and the SGD update graph (reference:
// include/frame/compiler/autograd.h:21-67; same names, signatures and output layout). Both are graph -> graph
// transformations called explicitly while building a training step; neither is a pipeline pass, so their results
// go through runtime::compile like any other graph.

#include <cstdint>
#include <span>

#include <frame/core/macros.h>
#include <frame/core/status.h>
#include <frame/ir/node.h>

namespace frame::ir {
class Graph;
}

namespace frame::compiler {

// Training graph = a clone of `forward` plus its backward nodes. Outputs: every forward output in its original
// order, then grad(forward.inputs()[wrt_input_indices[i]]) for each i in the given order.
// Errors: loss_output_index out of range, a non-scalar loss (rank 0 or numel 1 required), an out-of-range or
// repeated wrt index -> kInvalidArgument; an op on the loss's dependency chain without a GradientFn ->
// kUnimplemented; an op with OpTrait::kHasSideEffect on that chain -> kInvalidArgument. A wrt input that the loss
// does not depend on gets an all-zero constant gradient.
FRAME_API Result<ir::Graph> build_backward_graph(const ir::Graph& forward, int32_t loss_output_index,
                                                 std::span<const int32_t> wrt_input_indices);

// SGD step as its own graph: inputs [param_0..param_{n-1}, grad_0..grad_{n-1}], outputs
// new_param_i = add(param_i, mul(constant(-learning_rate), grad_i)), the constant splatted to param_i's shape.
// Errors (kInvalidArgument): empty param_types, non-finite learning_rate, a dtype outside float32/float16/bfloat16.
FRAME_API Result<ir::Graph> build_sgd_update_graph(std::span<const ir::TensorType> param_types, double learning_rate);

}  // namespace frame::compiler

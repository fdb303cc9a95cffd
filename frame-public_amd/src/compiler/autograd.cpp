// Reverse-mode differentiation over the IR (reference: src/compiler/autograd.cpp:118-450). The training graph is
// built in the same node order as the reference's (clone, seed, then per forward node in reverse topological order:
// its gradient micrograph, then one accumulating add per already-seen input), so its IR text is identical.
#include <frame/compiler/autograd.h>

#include <cmath>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include <frame/ir/graph.h>
#include <frame/ops/constant_utils.h>
#include <frame/ops/graph_builder.h>
#include <frame/ops/op_registry.h>

namespace frame::compiler {

namespace {

using ValueMap = std::unordered_map<const ir::Value*, ir::Value*>;

Status internal(const std::string& msg) {
  return Status::make(ErrorCode::kInternal, "compiler::build_backward_graph: " + msg);
}

// Splices `micro` into `training`: micro's graph inputs stand for `bound` (positionally), every other node is
// re-created with its already-typed outputs and its attributes. Returns the training values of micro's outputs.
Result<std::vector<ir::Value*>> splice(ir::Graph& training, const ir::Graph& micro, const std::vector<ir::Value*>& bound) {
  if (micro.inputs().size() != bound.size())
    return internal("gradient micrograph declared " + std::to_string(micro.inputs().size()) + " graph input(s), expected " +
                    std::to_string(bound.size()));
  ValueMap map;
  for (size_t i = 0; i < bound.size(); ++i) map.emplace(micro.inputs()[i], bound[i]);
  for (const ir::Node* m : micro.topological_order()) {
    if (m->op() == ir::kGraphInputOp) continue;
    std::vector<ir::Value*> ins;
    for (const ir::Value* v : m->inputs()) {
      auto it = map.find(v);
      if (it == map.end()) return internal("gradient micrograph sub-op '" + std::string(m->op()) + "' input value has no mapping");
      ins.push_back(it->second);
    }
    std::vector<ir::TensorType> types;
    for (const ir::Value& o : m->outputs()) types.push_back(o.type());
    Result<ir::Node*> n = training.create_node(std::string(m->op()), std::move(ins), std::move(types));
    if (!n.is_ok()) return n.status();
    for (const auto& [k, v] : m->attrs()) n.value()->set_attr(k, v);
    for (size_t j = 0; j < m->outputs().size(); ++j) map.emplace(&m->outputs()[j], n.value()->output(static_cast<int32_t>(j)));
  }
  std::vector<ir::Value*> out;
  for (const ir::Value* v : micro.outputs()) {
    auto it = map.find(v);
    if (it == map.end()) return internal("gradient micrograph output value has no mapping");
    out.push_back(it->second);
  }
  return out;
}

// grad[value] += contribution (an `add` node once a second contribution arrives).
Status accumulate(ir::Graph& training, ValueMap& grad, const ir::Value* value, ir::Value* contribution) {
  auto [it, fresh] = grad.try_emplace(value, contribution);
  if (fresh) return Status::ok();
  Result<ir::Node*> sum = ops::create_node_with_inferred_types(training, "add", {it->second, contribution});
  if (!sum.is_ok()) return sum.status();
  it->second = sum.value()->output(0);
  return Status::ok();
}

Result<ir::Node*> splat(ir::Graph& g, const ir::TensorType& t, double v) {
  const ops::AttrMap attrs{{"value", std::vector<double>(static_cast<size_t>(t.shape.numel()), v)},
                           {"shape", t.shape},
                           {"dtype", t.dtype}};
  return ops::create_node_with_inferred_types(g, ops::kConstantOpName, t.device, attrs);
}

}  // namespace

Result<ir::Graph> build_backward_graph(const ir::Graph& forward, int32_t loss_output_index,
                                       std::span<const int32_t> wrt_input_indices) {
  const int32_t n_out = static_cast<int32_t>(forward.outputs().size());
  if (loss_output_index < 0 || loss_output_index >= n_out)
    return Status::make(ErrorCode::kInvalidArgument, "compiler::build_backward_graph: loss_output_index " +
                                                         std::to_string(loss_output_index) + " is out of range [0, " +
                                                         std::to_string(n_out) + ")");
  const ir::Value* loss_fwd = forward.outputs()[static_cast<size_t>(loss_output_index)];
  const Shape& ls = loss_fwd->type().shape;
  if (!(ls.rank() == 0 || ls.numel() == 1))
    return Status::make(ErrorCode::kInvalidArgument,
                        "compiler::build_backward_graph: loss output must be scalar (rank 0 or numel==1), got shape " +
                            ls.to_string());
  const int32_t n_in = static_cast<int32_t>(forward.inputs().size());
  std::unordered_set<int32_t> seen;
  for (int32_t idx : wrt_input_indices) {
    if (idx < 0 || idx >= n_in)
      return Status::make(ErrorCode::kInvalidArgument, "compiler::build_backward_graph: wrt_input_indices entry " +
                                                           std::to_string(idx) + " is out of range [0, " +
                                                           std::to_string(n_in) + ")");
    if (!seen.insert(idx).second)
      return Status::make(ErrorCode::kInvalidArgument,
                          "compiler::build_backward_graph: wrt_input_indices entry " + std::to_string(idx) + " is duplicated");
  }

  ValueMap clone_map;
  Result<ir::Graph> cloned = ir::clone_graph(forward, &clone_map);
  if (!cloned.is_ok()) return cloned.status();
  ir::Graph training = std::move(cloned.value());
  ir::Value* loss = clone_map.at(loss_fwd);

  // Nodes the loss depends on: walk the (pre-backward) topological order backwards from the loss's producer.
  const std::vector<ir::Node*> order = training.topological_order();
  std::unordered_set<const ir::Node*> chain{loss->producer()};
  for (auto it = order.rbegin(); it != order.rend(); ++it)
    if (chain.count(*it) != 0)
      for (const ir::Value* v : (*it)->inputs()) chain.insert(v->producer());

  ValueMap grad;
  Result<ir::Node*> seed = splat(training, loss->type(), 1.0);
  if (!seed.is_ok()) return seed.status();
  FRAME_RETURN_IF_ERROR(accumulate(training, grad, loss, seed.value()->output(0)));

  for (auto it = order.rbegin(); it != order.rend(); ++it) {
    ir::Node* node = *it;
    if (chain.count(node) == 0 || node->inputs().empty()) continue;
    const std::string op(node->op());
    const ops::OpSchema* schema = ops::OpRegistry::instance().find(op);
    if (schema == nullptr) return internal("op '" + op + "' is not registered");
    if (schema->has_trait(ops::OpTrait::kHasSideEffect))
      return Status::make(ErrorCode::kInvalidArgument, "compiler::build_backward_graph: op '" + op +
                                                           "' has OpTrait::kHasSideEffect and cannot appear on the loss "
                                                           "dependency chain");
    if (schema->gradient() == nullptr)
      return Status::make(ErrorCode::kUnimplemented,
                          "compiler::build_backward_graph: op '" + op + "' has no registered GradientFn");
    std::vector<ir::Value*> gys;
    for (size_t j = 0; j < node->outputs().size(); ++j) {
      auto g = grad.find(&node->outputs()[j]);
      if (g == grad.end())
        return internal("op '" + op + "' output has no accumulated gradient despite being on the loss dependency chain");
      gys.push_back(g->second);
    }
    ops::NodeContext ctx;
    ctx.op = node->op();
    for (const ir::Value* v : node->inputs()) ctx.input_types.push_back(v->type());
    ctx.attrs = &node->attrs();
    Result<ir::Graph> micro = schema->gradient()(ctx);
    if (!micro.is_ok())
      return Status::make(micro.status().code(), "compiler::build_backward_graph: op '" + op +
                                                     "' GradientFn failed: " + std::string(micro.status().message()));
    const size_t n = node->inputs().size(), m = node->outputs().size();
    if (micro.value().inputs().size() != n + 2 * m)
      return internal("op '" + op + "' gradient micrograph declared " + std::to_string(micro.value().inputs().size()) +
                      " graph input(s), expected " + std::to_string(n + 2 * m) + " ([x.., y.., gy..])");
    if (micro.value().outputs().size() != n)
      return Status::make(ErrorCode::kInvalidArgument,
                          "compiler::build_backward_graph: op '" + op + "' gradient micrograph produced " +
                              std::to_string(micro.value().outputs().size()) + " graph output(s), expected " +
                              std::to_string(n) + " (one gradient per input)");
    std::vector<ir::Value*> bound(node->inputs().begin(), node->inputs().end());
    for (size_t j = 0; j < m; ++j) bound.push_back(node->output(static_cast<int32_t>(j)));
    bound.insert(bound.end(), gys.begin(), gys.end());
    Result<std::vector<ir::Value*>> gx = splice(training, micro.value(), bound);
    if (!gx.is_ok()) return gx.status();
    for (size_t i = 0; i < n; ++i) FRAME_RETURN_IF_ERROR(accumulate(training, grad, node->inputs()[i], gx.value()[i]));
  }

  for (int32_t idx : wrt_input_indices) {
    ir::Value* x = clone_map.at(forward.inputs()[static_cast<size_t>(idx)]);
    auto g = grad.find(x);
    ir::Value* out = nullptr;
    if (g != grad.end()) {
      out = g->second;
    } else {
      Result<ir::Node*> zero = splat(training, x->type(), 0.0);
      if (!zero.is_ok()) return zero.status();
      out = zero.value()->output(0);
    }
    FRAME_RETURN_IF_ERROR(training.mark_output(out));
  }
  return training;
}

Result<ir::Graph> build_sgd_update_graph(std::span<const ir::TensorType> param_types, double learning_rate) {
  if (param_types.empty())
    return Status::make(ErrorCode::kInvalidArgument, "compiler::build_sgd_update_graph: param_types must not be empty");
  if (!std::isfinite(learning_rate))
    return Status::make(ErrorCode::kInvalidArgument, "compiler::build_sgd_update_graph: learning_rate must be finite, got " +
                                                         std::to_string(learning_rate));
  for (size_t i = 0; i < param_types.size(); ++i)
    if (!ops::is_constant_dtype_supported(param_types[i].dtype))
      return Status::make(ErrorCode::kInvalidArgument, "compiler::build_sgd_update_graph: param_types[" + std::to_string(i) +
                                                           "] has unsupported dtype '" +
                                                           std::string(param_types[i].dtype.name()) +
                                                           "' (v0 supports float32/float16/bfloat16 only)");
  ir::Graph g("sgd_update");
  std::vector<ir::Value*> params, grads;
  for (const ir::TensorType& t : param_types) {
    Result<ir::Value*> v = g.add_graph_input(t);
    if (!v.is_ok()) return v.status();
    params.push_back(v.value());
  }
  for (const ir::TensorType& t : param_types) {
    Result<ir::Value*> v = g.add_graph_input(t);
    if (!v.is_ok()) return v.status();
    grads.push_back(v.value());
  }
  for (size_t i = 0; i < param_types.size(); ++i) {
    Result<ir::Node*> lr = splat(g, param_types[i], -learning_rate);
    if (!lr.is_ok()) return lr.status();
    Result<ir::Node*> step = ops::create_node_with_inferred_types(g, "mul", {lr.value()->output(0), grads[i]});
    if (!step.is_ok()) return step.status();
    Result<ir::Node*> upd = ops::create_node_with_inferred_types(g, "add", {params[i], step.value()->output(0)});
    if (!upd.is_ok()) return upd.status();
    FRAME_RETURN_IF_ERROR(g.mark_output(upd.value(), 0));
  }
  return g;
}

}  // namespace frame::compiler

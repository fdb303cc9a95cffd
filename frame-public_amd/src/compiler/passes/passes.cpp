// The nine standard passes (reference behaviour: src/compiler/passes/*.cpp).
//
// Two deliberate differences from the reference, both because this library ships no `cpu` backend (the CPU
// reference lives only in the test oracle):
//  * constant_folding evaluates foldable nodes with a small host evaluator of its own (fp32 arithmetic, one
//    round-to-nearest-even per node, exactly the CPU semantics) instead of borrowing the cpu backend's
//    kernels (reference: src/compiler/passes/constant_folding.cpp:60-150).
//  * operator_fusion requires every chain member to have a kernel on the graph's target backend, where the
//    reference asks for a cpu kernel (reference: src/compiler/passes/operator_fusion.cpp:150-158). For cpu
//    graphs the two rules coincide.
#include <algorithm>
#include <cmath>
#include <map>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

#include <frame/compiler/pass.h>
#include <frame/core/device.h>
#include <frame/hal/backend.h>
#include <frame/ir/graph.h>
#include <frame/ir/memory_plan.h>
#include <frame/ir/serialization.h>
#include <frame/ops/constant_utils.h>
#include <frame/ops/fused_elementwise_utils.h>
#include <frame/ops/kernel_registry.h>
#include <frame/ops/op_registry.h>

namespace frame::compiler {
namespace {

const ops::OpSchema* schema_of(const ir::Node* n) { return ops::OpRegistry::instance().find(n->op()); }
bool has(const ir::Node* n, ops::OpTrait t) {
  const ops::OpSchema* s = schema_of(n);
  return s != nullptr && s->has_trait(t);
}
bool is_constant(const ir::Node* n) { return n != nullptr && n->op() == ops::kConstantOpName; }

// ---- canonicalize: commutative binary ops take a constant operand on the right ------------------------------
class CanonicalizePass final : public PassBase<CanonicalizePass> {
 public:
  static constexpr std::string_view kName = "canonicalize";
  Status run_impl(ir::Graph& g) {
    for (ir::Node* n : g.topological_order()) {
      if (n->inputs().size() != 2 || !has(n, ops::OpTrait::kCommutative)) continue;
      if (is_constant(n->inputs()[0]->producer()) && !is_constant(n->inputs()[1]->producer()))
        FRAME_RETURN_IF_ERROR(g.swap_node_inputs(n, 0, 1));
    }
    return Status::ok();
  }
};

// ---- shape_inference: validate stored output types against the schemas ------------------------------------
class ShapeInferencePass final : public PassBase<ShapeInferencePass> {
 public:
  static constexpr std::string_view kName = "shape_inference";
  Status run_impl(ir::Graph& g) {
    for (ir::Node* n : g.topological_order()) {
      if (n->op() == ir::kGraphInputOp) continue;
      const std::string op(n->op());
      const ops::OpSchema* s = schema_of(n);
      if (s == nullptr) return Status::make(ErrorCode::kNotFound, "shape_inference: op '" + op + "' is not registered");
      if (s->shape_infer() == nullptr)
        return Status::make(ErrorCode::kInvalidArgument, "shape_inference: op '" + op + "' has no shape_infer function registered");
      ops::NodeContext ctx;
      ctx.op = n->op();
      for (const ir::Value* in : n->inputs()) ctx.input_types.push_back(in->type());
      ctx.attrs = &n->attrs();
      Result<std::vector<Shape>> shapes = s->shape_infer()(ctx);
      if (!shapes.is_ok())
        return Status::make(shapes.status().code(), "shape_inference: node '" + op + "' shape_infer failed: " +
                                                        std::string(shapes.status().message()));
      if (shapes.value().size() != n->outputs().size())
        return Status::make(ErrorCode::kInvalidArgument, "shape_inference: node '" + op + "' shape_infer returned " +
                                                             std::to_string(shapes.value().size()) + " shape(s), node has " +
                                                             std::to_string(n->outputs().size()) + " output(s)");
      for (size_t i = 0; i < n->outputs().size(); ++i) {
        const ir::TensorType& t = n->outputs()[i].type();
        if (!(shapes.value()[i] == t.shape))
          return Status::make(ErrorCode::kInvalidArgument, "shape_inference: node '" + op + "' output " + std::to_string(i) +
                                                               " shape mismatch: inferred " + shapes.value()[i].to_string() +
                                                               ", existing " + t.shape.to_string());
        if (!n->inputs().empty() && !(t.dtype == ctx.input_types[0].dtype))
          return Status::make(ErrorCode::kInvalidArgument,
                              "shape_inference: node '" + op + "' output " + std::to_string(i) + " dtype '" +
                                  std::string(t.dtype.name()) + "' does not match input 0 dtype '" +
                                  std::string(ctx.input_types[0].dtype.name()) + "'");
      }
    }
    for (const ir::Node* n : g.topological_order())
      for (size_t i = 0; i < n->outputs().size(); ++i)
        if (n->outputs()[i].type().shape.has_dynamic_dim())
          return Status::make(ErrorCode::kInvalidArgument, "shape_inference: node '" + std::string(n->op()) + "' output " +
                                                               std::to_string(i) + " has a dynamic dimension, static shape required");
    return Status::ok();
  }
};

// ---- constant_folding --------------------------------------------------------------------------------------
// Host evaluation of one elementwise op on float payloads (inputs already widened from the constant's dtype).
bool fold_scalar(std::string_view op, const std::vector<float>& in, float& out) {
  if (op == "add") out = in[0] + in[1];
  else if (op == "mul") out = in[0] * in[1];
  else if (op == "relu") out = std::max(in[0], 0.0f);
  else if (op == "square") out = in[0] * in[0];
  else if (op == "gelu") out = 0.5f * in[0] * (1.0f + std::erf(in[0] * 0.70710678118654752440f));
  else if (op == "sigmoid") out = in[0] >= 0.0f ? 1.0f / (1.0f + std::exp(-in[0])) : std::exp(in[0]) / (1.0f + std::exp(in[0]));
  else if (op == "tanh") out = std::tanh(in[0]);
  else if (op == "rsqrt") out = 1.0f / std::sqrt(in[0]);
  else return false;
  return true;
}

float round_to(DType d, float v) {
  if (d.code() == DTypeCode::kBFloat16) return bfloat16_to_float(float_to_bfloat16(v));
  if (d.code() == DTypeCode::kFloat16) return float16_to_float(float_to_float16(v));
  return v;
}

class ConstantFoldingPass final : public PassBase<ConstantFoldingPass> {
 public:
  static constexpr std::string_view kName = "constant_folding";
  Status run_impl(ir::Graph& g) {
    const std::vector<ir::Node*> snapshot = g.topological_order();
    for (ir::Node* n : snapshot) {
      if (is_constant(n) || n->outputs().size() != 1 || n->inputs().empty()) continue;
      const ops::OpSchema* s = schema_of(n);
      if (s == nullptr || s->has_trait(ops::OpTrait::kHasSideEffect) || !s->has_trait(ops::OpTrait::kElementwise)) continue;
      if (!std::all_of(n->inputs().begin(), n->inputs().end(), [](const ir::Value* v) { return is_constant(v->producer()); }))
        continue;
      const ir::TensorType out_t = n->outputs()[0].type();
      const DTypeCode c = out_t.dtype.code();
      if (c != DTypeCode::kFloat32 && c != DTypeCode::kFloat16 && c != DTypeCode::kBFloat16) continue;
      std::vector<const std::vector<double>*> payload;
      for (const ir::Value* v : n->inputs()) payload.push_back(v->producer()->attr<std::vector<double>>("value"));
      if (std::any_of(payload.begin(), payload.end(), [](auto* p) { return p == nullptr; })) continue;
      const size_t numel = static_cast<size_t>(out_t.shape.numel());
      std::vector<double> folded(numel);
      bool ok = true;
      std::vector<float> args(payload.size());
      for (size_t i = 0; i < numel && ok; ++i) {
        for (size_t a = 0; a < payload.size(); ++a) args[a] = round_to(out_t.dtype, static_cast<float>((*payload[a])[i]));
        float r = 0;
        ok = fold_scalar(n->op(), args, r);
        folded[i] = round_to(out_t.dtype, r);
      }
      if (!ok) continue;  // not an op this evaluator knows: leave it to the backend
      Result<ir::Node*> cn = g.create_node(std::string(ops::kConstantOpName), {}, {out_t});
      if (!cn.is_ok()) return cn.status();
      cn.value()->set_attr("value", ir::AttrValue{std::move(folded)});
      cn.value()->set_attr("shape", ir::AttrValue{out_t.shape});
      cn.value()->set_attr("dtype", ir::AttrValue{out_t.dtype});
      FRAME_RETURN_IF_ERROR(g.replace_all_uses(n->output(0), cn.value()->output(0)));
      FRAME_RETURN_IF_ERROR(g.erase_node(n));
    }
    return Status::ok();
  }
};

// ---- common_subexpression_elimination ----------------------------------------------------------------------
class CsePass final : public PassBase<CsePass> {
 public:
  static constexpr std::string_view kName = "common_subexpression_elimination";
  Status run_impl(ir::Graph& g) {
    const std::vector<ir::Node*> snapshot = g.topological_order();
    std::unordered_map<const ir::Node*, int64_t> index;
    for (size_t i = 0; i < snapshot.size(); ++i) index[snapshot[i]] = static_cast<int64_t>(i);
    std::unordered_map<std::string, ir::Node*> seen;
    for (ir::Node* n : snapshot) {
      if (n->op() == ir::kGraphInputOp) continue;
      const ops::OpSchema* s = schema_of(n);
      if (s == nullptr || s->has_trait(ops::OpTrait::kHasSideEffect)) continue;
      std::vector<std::pair<int64_t, int32_t>> ins;
      for (const ir::Value* v : n->inputs()) ins.emplace_back(index.at(v->producer()), v->output_index());
      if (s->has_trait(ops::OpTrait::kCommutative) && ins.size() == 2 && ins[1] < ins[0]) std::swap(ins[0], ins[1]);
      std::string key(n->op());
      key += '|';
      for (auto [p, o] : ins) key += std::to_string(p) + ":" + std::to_string(o) + ",";
      key += '|';
      std::map<std::string, const ir::AttrValue*> sorted;
      for (const auto& [k, v] : n->attrs()) sorted.emplace(k, &v);
      for (const auto& [k, v] : sorted) key += k + "=" + ir::format_attr_value(*v) + ";";
      auto [it, fresh] = seen.try_emplace(std::move(key), n);
      if (fresh) continue;
      for (int32_t i = 0; i < static_cast<int32_t>(n->outputs().size()); ++i)
        FRAME_RETURN_IF_ERROR(g.replace_all_uses(n->output(i), it->second->output(i)));
      FRAME_RETURN_IF_ERROR(g.erase_node(n));
    }
    return Status::ok();
  }
};

// ---- dead_node_elimination ---------------------------------------------------------------------------------
class DnePass final : public PassBase<DnePass> {
 public:
  static constexpr std::string_view kName = "dead_node_elimination";
  Status run_impl(ir::Graph& g) {
    std::unordered_set<const ir::Node*> live;
    std::vector<const ir::Node*> work;
    auto mark = [&](const ir::Node* n) {
      if (n != nullptr && live.insert(n).second) work.push_back(n);
    };
    for (const ir::Value* v : g.outputs()) mark(v->producer());
    for (const ir::Node* n : g.topological_order())
      if (has(n, ops::OpTrait::kHasSideEffect)) mark(n);
    while (!work.empty()) {
      const ir::Node* n = work.back();
      work.pop_back();
      for (const ir::Value* in : n->inputs()) mark(in->producer());
    }
    const std::vector<ir::Node*> snapshot = g.topological_order();
    for (auto it = snapshot.rbegin(); it != snapshot.rend(); ++it)
      if ((*it)->op() != ir::kGraphInputOp && !live.count(*it)) FRAME_RETURN_IF_ERROR(g.erase_node(*it));
    return Status::ok();
  }
};

// ---- layout_assignment: every value is row-major ------------------------------------------------------------
class LayoutAssignmentPass final : public PassBase<LayoutAssignmentPass> {
 public:
  static constexpr std::string_view kName = "layout_assignment";
  Status run_impl(ir::Graph& g) {
    for (ir::Node* n : g.topological_order())
      for (int32_t i = 0; i < static_cast<int32_t>(n->outputs().size()); ++i)
        FRAME_RETURN_IF_ERROR(g.assign_layout(n->output(i), ir::Layout::kRowMajor));
    return Status::ok();
  }
};

// ---- operator_fusion: linear chains (>= 2) of attribute-free elementwise+fusable single-output nodes ----------
bool fusable(const ir::Node* n) {
  return has(n, ops::OpTrait::kElementwise) && has(n, ops::OpTrait::kFusable) && n->attrs().empty() &&
         n->outputs().size() == 1;
}

class OperatorFusionPass final : public PassBase<OperatorFusionPass> {
 public:
  static constexpr std::string_view kName = "operator_fusion";
  Status run_impl(ir::Graph& g) {
    const std::vector<ir::Node*> snapshot = g.topological_order();
    const std::unordered_set<const ir::Value*> outs(g.outputs().begin(), g.outputs().end());
    std::unordered_map<const ir::Value*, std::vector<ir::Node*>> users;
    for (ir::Node* n : snapshot)
      for (ir::Value* in : n->inputs()) users[in].push_back(n);
    std::unordered_set<const ir::Node*> done;
    for (ir::Node* head : snapshot) {
      if (!done.insert(head).second || !fusable(head)) continue;
      std::vector<ir::Node*> chain{head};
      for (;;) {
        const ir::Value* tail = chain.back()->output(0);
        if (outs.count(tail)) break;
        auto u = users.find(tail);
        if (u == users.end() || u->second.size() != 1) break;
        ir::Node* next = u->second[0];
        if (done.count(next) || !fusable(next) || next->inputs().empty() || next->inputs()[0] != tail) break;
        chain.push_back(next);
        done.insert(next);
      }
      if (chain.size() < 2) continue;
      const std::string_view backend = head->outputs()[0].type().device.backend;
      if (!std::all_of(chain.begin(), chain.end(), [&](const ir::Node* m) {
            return ops::KernelRegistry::instance().find(m->op(), backend).is_ok();
          }))
        continue;
      FRAME_RETURN_IF_ERROR(fuse(g, chain));
    }
    return Status::ok();
  }

 private:
  static Status fuse(ir::Graph& g, const std::vector<ir::Node*>& chain) {
    std::vector<ir::Value*> ext;
    std::vector<std::string> names;
    std::vector<int64_t> arities;
    for (size_t i = 0; i < chain.size(); ++i) {
      names.emplace_back(chain[i]->op());
      arities.push_back(static_cast<int64_t>(chain[i]->inputs().size()));
      for (size_t j = (i == 0 ? 0 : 1); j < chain[i]->inputs().size(); ++j) ext.push_back(chain[i]->inputs()[j]);
    }
    ir::Node* tail = chain.back();
    Result<ir::Node*> f = g.create_node(std::string(ops::kFusedElementwiseOpName), ext, {tail->output(0)->type()});
    if (!f.is_ok()) return f.status();
    std::unordered_map<std::string, ir::AttrValue> attrs;
    ops::encode_fused_chain(names, arities, attrs);
    for (auto& [k, v] : attrs) f.value()->set_attr(k, std::move(v));
    FRAME_RETURN_IF_ERROR(g.replace_all_uses(tail->output(0), f.value()->output(0)));
    for (auto it = chain.rbegin(); it != chain.rend(); ++it) FRAME_RETURN_IF_ERROR(g.erase_node(*it));
    return Status::ok();
  }
};

// ---- memory_planning: the graph must be plannable -----------------------------------------------------------
class MemoryPlanningPass final : public PassBase<MemoryPlanningPass> {
 public:
  static constexpr std::string_view kName = "memory_planning";
  Status run_impl(ir::Graph& g) {
    Result<ir::MemoryPlan> p = ir::compute_memory_plan(g);
    return p.is_ok() ? Status::ok() : p.status();
  }
};

// ---- backend_lowering: every node must have a kernel on the target backend ----------------------------------
class BackendLoweringPass final : public PassBase<BackendLoweringPass> {
 public:
  static constexpr std::string_view kName = "backend_lowering";
  Status run_impl(ir::Graph& g) {
    const auto& topo = g.topological_order();
    if (std::all_of(topo.begin(), topo.end(), [](const ir::Node* n) { return n->op() == ir::kGraphInputOp; }))
      return Status::ok();
    std::string_view backend;
    bool found = false;
    for (const ir::Node* n : topo)
      if (!n->outputs().empty()) {
        backend = n->outputs()[0].type().device.backend;
        found = true;
        break;
      }
    if (!found)
      return Status::make(ErrorCode::kInternal,
                          "backend_lowering: graph has operator node(s) but no Value carries a device, cannot determine target backend");
    Result<hal::Backend*> b = hal::BackendRegistry::instance().get(backend);
    if (!b.is_ok()) return Status::make(b.status().code(), "backend_lowering: " + std::string(b.status().message()));
    for (const ir::Node* n : topo) {
      if (n->op() == ir::kGraphInputOp) continue;
      Result<ops::KernelFn> k = ops::KernelRegistry::instance().find(n->op(), backend);
      if (!k.is_ok()) return Status::make(ErrorCode::kUnimplemented, "backend_lowering: " + std::string(k.status().message()));
    }
    return Status::ok();
  }
};

}  // namespace

FRAME_REGISTER_PASS(CanonicalizePass);
FRAME_REGISTER_PASS(ShapeInferencePass);
FRAME_REGISTER_PASS(ConstantFoldingPass);
FRAME_REGISTER_PASS(CsePass);
FRAME_REGISTER_PASS(DnePass);
FRAME_REGISTER_PASS(LayoutAssignmentPass);
FRAME_REGISTER_PASS(OperatorFusionPass);
FRAME_REGISTER_PASS(MemoryPlanningPass);
FRAME_REGISTER_PASS(BackendLoweringPass);

}  // namespace frame::compiler

// build_executable_plan (reference: src/ops/executable_plan.cpp:16-121) and the fused-chain codec
// (reference: src/ops/fused_elementwise_utils.cpp:17-206).
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include <frame/core/tensor.h>
#include <frame/ir/graph.h>
#include <frame/ir/memory_plan.h>
#include <frame/ops/executable_plan.h>
#include <frame/ops/fused_elementwise_utils.h>
#include <frame/ops/op_registry.h>

namespace frame::ops {

Result<ExecutablePlan> build_executable_plan(const ir::Graph& graph, std::string_view backend) {
  Result<ir::MemoryPlan> mem = ir::compute_memory_plan(graph);
  if (!mem.is_ok())
    return Status::make(mem.status().code(), "build_executable_plan: " + std::string(mem.status().message()));
  ExecutablePlan plan;
  plan.arena_total_bytes = mem.value().total_bytes;
  std::unordered_map<const ir::Value*, int32_t> slot;
  int32_t next = 0;
  for (const ir::Value* in : graph.inputs()) {
    slot.emplace(in, next++);
    plan.input_types.push_back(in->type());
  }
  const auto& topo = graph.topological_order();
  for (size_t t = 0; t < topo.size(); ++t) {
    const ir::Node* n = topo[t];
    if (n->op() == ir::kGraphInputOp) continue;
    Result<KernelFn> k = KernelRegistry::instance().find(n->op(), backend);
    if (!k.is_ok())
      return Status::make(ErrorCode::kUnimplemented, "build_executable_plan: " + std::string(k.status().message()));
    ExecutablePlanStep step;
    step.op = std::string(n->op());
    step.kernel = k.value();
    step.attrs = n->attrs();
    for (const ir::Value* in : n->inputs()) {
      auto it = slot.find(in);
      if (it == slot.end())
        return Status::make(ErrorCode::kInternal, "build_executable_plan: input value has no assigned slot for node '" +
                                                      step.op + "' (violates topological order invariant)");
      step.input_slots.push_back(it->second);
    }
    for (size_t j = 0; j < n->outputs().size(); ++j) {
      const ir::Value& out = n->outputs()[j];
      slot.emplace(&out, next);
      step.output_slots.push_back(next++);
      step.output_types.push_back(out.type());
      auto e = mem.value().entries.find({static_cast<int64_t>(t), static_cast<int32_t>(j)});
      step.output_arena_offsets.push_back(e == mem.value().entries.end() ? std::nullopt
                                                                        : std::optional<size_t>(e->second.byte_offset));
    }
    plan.steps.push_back(std::move(step));
  }
  plan.slot_count = next;
  for (const ir::Value* out : graph.outputs()) {
    auto it = slot.find(out);
    if (it == slot.end())
      return Status::make(ErrorCode::kInternal, "build_executable_plan: graph output value has no assigned slot");
    plan.output_types.push_back(out->type());
    plan.output_slots.push_back(it->second);
  }
  return plan;
}

void encode_fused_chain(const std::vector<std::string>& ops, const std::vector<int64_t>& arities,
                        std::unordered_map<std::string, ir::AttrValue>& attrs) {
  FRAME_CHECK(!ops.empty() && ops.size() == arities.size());
  std::string joined;
  for (const std::string& op : ops) joined += (joined.empty() ? "" : ";") + op;
  attrs["ops"] = ir::AttrValue{std::move(joined)};
  attrs["arities"] = ir::AttrValue{arities};
}

Status decode_and_validate_fused_chain(const std::unordered_map<std::string, ir::AttrValue>& attrs,
                                       int64_t expected_input_count, FusedElementwiseChain& out) {
  const std::string self(kFusedElementwiseOpName);
  auto bad = [&](const std::string& m) { return Status::make(ErrorCode::kInvalidArgument, "op '" + self + "' " + m); };
  auto ops_it = attrs.find("ops");
  if (ops_it == attrs.end()) return bad("is missing required attribute 'ops' (string)");
  const std::string* joined = std::get_if<std::string>(&ops_it->second);
  if (joined == nullptr) return bad("attribute 'ops' has wrong type, expected string");
  auto ar_it = attrs.find("arities");
  if (ar_it == attrs.end()) return bad("is missing required attribute 'arities' (int64 array)");
  const std::vector<int64_t>* arities = std::get_if<std::vector<int64_t>>(&ar_it->second);
  if (arities == nullptr) return bad("attribute 'arities' has wrong type, expected int64 array");
  std::vector<std::string> subs;
  for (size_t start = 0;;) {
    const size_t sep = joined->find(';', start);
    subs.push_back(joined->substr(start, sep == std::string::npos ? std::string::npos : sep - start));
    if (sep == std::string::npos) break;
    start = sep + 1;
  }
  if (subs.size() != arities->size())
    return bad("attribute 'ops' has " + std::to_string(subs.size()) + " segment(s), attribute 'arities' has " +
               std::to_string(arities->size()) + " element(s), expected equal counts");
  int64_t sum = 0;
  for (int64_t a : *arities) sum += a;
  const int64_t computed = sum - static_cast<int64_t>(subs.size() - 1);
  if (computed != expected_input_count)
    return bad("arities are inconsistent with input count: sum(arities)=" + std::to_string(sum) + ", segment count=" +
               std::to_string(subs.size()) + ", computed input count=" + std::to_string(computed) + ", expected " +
               std::to_string(expected_input_count));
  for (const std::string& sub : subs) {
    const OpSchema* s = OpRegistry::instance().find(sub);
    if (s == nullptr)
      return Status::make(ErrorCode::kNotFound, "op '" + self + "' sub-op '" + sub + "' is not registered");
    if (!s->has_trait(OpTrait::kElementwise) || !s->has_trait(OpTrait::kFusable))
      return bad("sub-op '" + sub + "' must have both kElementwise and kFusable traits");
  }
  out.sub_ops = std::move(subs);
  out.arities = *arities;
  return Status::ok();
}

Status execute_fused_chain(const KernelContext& ctx, hal::Allocator& allocator) {
  const std::string self(kFusedElementwiseOpName);
  if (ctx.outputs.size() != 1)
    return Status::make(ErrorCode::kInvalidArgument,
                        "op '" + self + "' expects 1 output, got " + std::to_string(ctx.outputs.size()));
  if (ctx.attrs == nullptr) return Status::make(ErrorCode::kInvalidArgument, "op '" + self + "' requires non-null attrs");
  FusedElementwiseChain chain;
  FRAME_RETURN_IF_ERROR(decode_and_validate_fused_chain(*ctx.attrs, static_cast<int64_t>(ctx.inputs.size()), chain));
  Tensor prev;
  size_t next_in = 0;
  for (size_t seg = 0; seg < chain.sub_ops.size(); ++seg) {
    std::vector<Tensor> ins;
    if (seg != 0) ins.push_back(prev);
    while (ins.size() < static_cast<size_t>(chain.arities[seg])) {
      if (next_in >= ctx.inputs.size())
        return Status::make(ErrorCode::kInternal, "op '" + self + "' sub-op '" + chain.sub_ops[seg] +
                                                      "' ran out of external inputs (violates arities self-consistency)");
      ins.push_back(ctx.inputs[next_in++]);
    }
    Tensor out;
    if (seg + 1 == chain.sub_ops.size()) {
      out = ctx.outputs[0];
    } else {
      Result<Tensor> t = Tensor::empty(ctx.outputs[0].shape(), ctx.outputs[0].dtype(), ctx.device, allocator);
      if (!t.is_ok()) return t.status();
      out = t.value();
    }
    Result<KernelFn> k = KernelRegistry::instance().find(chain.sub_ops[seg], ctx.device.backend);
    if (!k.is_ok()) return k.status();
    std::vector<Tensor> outs{out};
    KernelContext sub{ins, outs, nullptr, ctx.device, ctx.stream, ctx.compile_options};
    FRAME_RETURN_IF_ERROR(k.value()(sub));
    prev = out;
  }
  return Status::ok();
}

}  // namespace frame::ops

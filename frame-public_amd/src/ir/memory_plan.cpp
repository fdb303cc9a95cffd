// First-fit arena planning of intermediate values (algorithm and exclusions as in the reference,
// src/ir/memory_plan.cpp:160-256: values in topological order; a value may reuse space of every value whose
// last use is strictly before its definition; candidate offsets start at 0 and step past each live interval
// in address order, rounded up to 64 bytes).
#include <algorithm>
#include <limits>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include <frame/core/storage.h>
#include <frame/ir/graph.h>
#include <frame/ir/memory_plan.h>

namespace frame::ir {

Result<MemoryPlan> compute_memory_plan(const Graph& graph) {
  const std::unordered_set<const Value*> outputs(graph.outputs().begin(), graph.outputs().end());
  const auto& topo = graph.topological_order();

  struct Item {
    MemoryPlanKey key;
    size_t bytes;
    int64_t def, last;
  };
  std::vector<Item> items;
  std::unordered_map<const Value*, size_t> slot;
  for (size_t i = 0; i < topo.size(); ++i) {
    const Node* n = topo[i];
    if (n->op() == kGraphInputOp) continue;
    for (size_t j = 0; j < n->outputs().size(); ++j) {
      const Value* v = &n->outputs()[j];
      if (outputs.count(v)) continue;
      const TensorType& t = v->type();
      if (t.shape.has_dynamic_dim())
        return Status::make(ErrorCode::kInvalidArgument, "compute_memory_plan: node '" + std::string(n->op()) +
                                                             "' output " + std::to_string(j) +
                                                             " has a dynamic dimension, static shape required");
      const size_t numel = static_cast<size_t>(t.shape.numel());
      const size_t item = t.dtype.itemsize();
      if (item != 0 && numel > std::numeric_limits<size_t>::max() / item)
        return Status::make(ErrorCode::kInvalidArgument, "compute_memory_plan: node '" + std::string(n->op()) +
                                                             "' output " + std::to_string(j) + " size overflows size_t");
      slot.emplace(v, items.size());
      items.push_back({{static_cast<int64_t>(i), static_cast<int32_t>(j)}, numel * item, static_cast<int64_t>(i),
                       static_cast<int64_t>(i)});
    }
  }
  for (size_t i = 0; i < topo.size(); ++i)
    for (const Value* in : topo[i]->inputs()) {
      auto it = slot.find(in);
      if (it != slot.end()) items[it->second].last = std::max(items[it->second].last, static_cast<int64_t>(i));
    }

  struct Live {
    size_t begin, end;
    int64_t last;
  };
  std::vector<Live> live;
  MemoryPlan plan;
  for (const Item& it : items) {
    std::erase_if(live, [&](const Live& l) { return l.last < it.def; });
    std::sort(live.begin(), live.end(), [](const Live& a, const Live& b) { return a.begin < b.begin; });
    size_t at = 0;
    for (const Live& l : live) {
      if (at + it.bytes <= l.begin) break;
      at = (l.end + kDefaultAlignment - 1) / kDefaultAlignment * kDefaultAlignment;
    }
    plan.entries.emplace(it.key, MemoryPlanEntry{at, it.bytes, it.def, it.last});
    live.push_back({at, at + it.bytes, it.last});
    plan.total_bytes = std::max(plan.total_bytes, at + it.bytes);
  }
  return plan;
}

}  // namespace frame::ir

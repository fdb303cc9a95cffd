#pragma once
// ExecutablePlan: what every backend executor shares — the slot table (graph inputs then node outputs in
// topological order), one step per non-input node with its resolved KernelFn, the arena offsets of the memory
// plan, and the I/O types (reference: include/frame/ops/executable_plan.h:42-71).

#include <cstddef>
#include <cstdint>
#include <optional>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

#include <frame/core/macros.h>
#include <frame/core/status.h>
#include <frame/ir/attribute.h>
#include <frame/ir/node.h>
#include <frame/ops/kernel_registry.h>

namespace frame::ir {
class Graph;
}

namespace frame::ops {

struct ExecutablePlanStep {
  std::string op;
  KernelFn kernel = nullptr;
  std::unordered_map<std::string, ir::AttrValue> attrs;
  std::vector<int32_t> input_slots;
  std::vector<int32_t> output_slots;
  std::vector<ir::TensorType> output_types;
  std::vector<std::optional<size_t>> output_arena_offsets;  // nullopt = graph output (allocated separately)
};

struct ExecutablePlan {
  std::vector<ir::TensorType> input_types;
  std::vector<ir::TensorType> output_types;
  std::vector<int32_t> output_slots;
  std::vector<ExecutablePlanStep> steps;
  int32_t slot_count = 0;
  size_t arena_total_bytes = 0;
};

// A node without a kernel for `backend` yields kUnimplemented naming the op and the backend.
FRAME_API Result<ExecutablePlan> build_executable_plan(const ir::Graph& graph, std::string_view backend);

}  // namespace frame::ops

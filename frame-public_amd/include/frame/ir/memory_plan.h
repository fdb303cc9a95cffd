#pragma once
// Static memory plan of intermediate values: first-fit offsets in one arena, 64-byte aligned. Graph inputs and
// graph outputs are not planned (reference: include/frame/ir/memory_plan.h, src/ir/memory_plan.cpp:160-256).

#include <cstddef>
#include <cstdint>
#include <map>
#include <utility>

#include <frame/core/macros.h>
#include <frame/core/status.h>

namespace frame::ir {

class Graph;

struct MemoryPlanEntry {
  size_t byte_offset = 0;
  size_t size_bytes = 0;
  int64_t def_index = 0;       // topological index of the producer
  int64_t last_use_index = 0;  // largest topological index of a consumer (def_index when unused)
};

using MemoryPlanKey = std::pair<int64_t, int32_t>;  // (producer topological index, output index)

struct MemoryPlan {
  size_t total_bytes = 0;
  std::map<MemoryPlanKey, MemoryPlanEntry> entries;
};

FRAME_API Result<MemoryPlan> compute_memory_plan(const Graph& graph);

}  // namespace frame::ir

#pragma once
// OpRegistry: name -> OpSchema (reference: include/frame/ops/op_registry.h).

#include <string>
#include <string_view>
#include <unordered_map>

#include <frame/core/macros.h>
#include <frame/core/status.h>
#include <frame/ir/graph.h>
#include <frame/ops/op_schema.h>

namespace frame::ops {

class FRAME_API OpRegistry {
 public:
  static OpRegistry& instance() noexcept;
  // Aborts on an invalid, reserved or duplicate name (registration happens in static initialisers).
  OpSchema& register_op(std::string_view name) noexcept;
  const OpSchema* find(std::string_view name) const;

 private:
  std::unordered_map<std::string, OpSchema> schemas_;
};

// OpQuery for Graph::verify: V3 = op registered; V4 = input count (exact, or at least min_input_count() with a
// variadic group), output count, required attributes present, attribute types, no unknown attributes.
FRAME_API ir::OpQuery make_op_query();

}  // namespace frame::ops

#define FRAME_REGISTER_OP(name)                                                                 \
  [[maybe_unused]] static ::frame::ops::OpSchema& FRAME_CONCAT(frame_op_schema_, __COUNTER__) = \
      ::frame::ops::OpRegistry::instance().register_op(name)

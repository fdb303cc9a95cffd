#pragma once
// Graph: static SSA graph with nodes kept in topological order (reference: include/frame/ir/graph.h:50-187).
// Mutation goes through a small set of checked APIs used by compiler passes.

#include <functional>
#include <memory>
#include <string>
#include <string_view>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include <frame/core/macros.h>
#include <frame/core/status.h>
#include <frame/ir/node.h>

namespace frame::ir {

inline constexpr std::string_view kGraphInputOp = "graph_input";
inline constexpr std::string_view kGraphOutputMarker = "graph_output";

// ^[a-z][a-z0-9_]*$
FRAME_API bool matches_op_name_charset(std::string_view name) noexcept;

// Callbacks through which verify() consults the op registry (ir does not depend on ops).
struct OpQuery {
  std::function<bool(std::string_view op_name)> op_registered;
  std::function<Status(const Node& node)> check_schema;
};

class FRAME_API Graph {
 public:
  Graph() = default;
  explicit Graph(std::string name) : name_(std::move(name)) {}

  std::string_view name() const { return name_; }

  Result<Node*> create_node(std::string op, std::vector<Value*> inputs, std::vector<TensorType> output_types);
  Result<Value*> add_graph_input(TensorType type);
  Status mark_output(Value* value);
  Status mark_output(Node* node, int32_t output_index);
  Status erase_node(Node* node);
  // Rewrites every use of `from` (node inputs and graph outputs) to `to`; types must match. `to`'s producer
  // must precede `from`'s, or be movable to `from`'s position (all its inputs produced strictly earlier).
  Status replace_all_uses(Value* from, Value* to);
  Status swap_node_inputs(Node* node, int32_t i, int32_t j);
  Status assign_layout(Value* value, Layout layout);

  const std::vector<Node*>& topological_order() const { return topo_order_; }
  const std::vector<Value*>& inputs() const { return inputs_; }
  const std::vector<Value*>& outputs() const { return outputs_; }

  // Invariants V1..V7: SSA, acyclic, op registered, schema, static shapes/dtypes, one device, closed attrs.
  Status verify(const OpQuery& query) const;
  Status verify_structure() const;  // V1, V2, V5, V6, V7

 private:
  std::string name_;
  std::vector<std::unique_ptr<Node>> nodes_;
  std::vector<Node*> topo_order_;
  std::vector<Value*> inputs_;
  std::vector<Value*> outputs_;
  std::unordered_set<const Node*> node_set_;
};

// Rebuilds an equivalent independent graph through the public construction API (any backend name).
FRAME_API Result<Graph> clone_graph(const Graph& source,
                                    std::unordered_map<const Value*, Value*>* value_map = nullptr);

}  // namespace frame::ir

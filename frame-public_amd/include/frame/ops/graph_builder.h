#pragma once
// create_node_with_inferred_types: looks up the schema, runs its shape inference and creates the node with
// dtype/device taken from input 0 (or, for 0-input ops, the given device and the "dtype" attribute)
// (reference: include/frame/ops/graph_builder.h:36-46).

#include <string_view>
#include <unordered_map>
#include <vector>

#include <frame/core/device.h>
#include <frame/core/macros.h>
#include <frame/core/status.h>
#include <frame/ir/attribute.h>
#include <frame/ir/node.h>

namespace frame::ir {
class Graph;
}

namespace frame::ops {

using AttrMap = std::unordered_map<std::string, ir::AttrValue>;

FRAME_API Result<ir::Node*> create_node_with_inferred_types(ir::Graph& graph, std::string_view op,
                                                            std::vector<ir::Value*> inputs, const AttrMap& attrs = {});
FRAME_API Result<ir::Node*> create_node_with_inferred_types(ir::Graph& graph, std::string_view op, Device device,
                                                            const AttrMap& attrs = {});

}  // namespace frame::ops

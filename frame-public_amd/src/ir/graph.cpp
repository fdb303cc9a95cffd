// Graph IR: construction, checked mutation, invariants V1..V7 and clone
// (reference behaviour: src/ir/graph.cpp, include/frame/ir/graph.h:50-187).
#include <algorithm>
#include <cstdint>
#include <memory>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

#include <frame/ir/graph.h>

namespace frame::ir {

namespace {

Status invalid(std::string msg) { return Status::make(ErrorCode::kInvalidArgument, msg); }

std::string_view layout_name(Layout l) { return l == Layout::kRowMajor ? "kRowMajor" : "kUnknown"; }

std::string device_text(const Device& d) { return std::string(d.backend) + ":" + std::to_string(d.index); }

}  // namespace

// ---- attributes / nodes -----------------------------------------------------------------------------------

AttrType attr_type_of(const AttrValue& value) { return static_cast<AttrType>(value.index()); }

std::string_view attr_type_name(AttrType type) {
  switch (type) {
    case AttrType::kInt64: return "int64";
    case AttrType::kDouble: return "double";
    case AttrType::kString: return "string";
    case AttrType::kBool: return "bool";
    case AttrType::kInt64Array: return "int64_array";
    case AttrType::kDoubleArray: return "double_array";
    case AttrType::kDType: return "dtype";
    case AttrType::kShape: return "shape";
  }
  FRAME_CHECK(false);
  return {};
}

void Node::set_attr(std::string name, AttrValue value) { attrs_.insert_or_assign(std::move(name), std::move(value)); }

const AttrValue* Node::find_attr(std::string_view name) const {
  auto it = attrs_.find(std::string(name));
  return it == attrs_.end() ? nullptr : &it->second;
}

bool matches_op_name_charset(std::string_view name) noexcept {
  if (name.empty() || name[0] < 'a' || name[0] > 'z') return false;
  return std::all_of(name.begin() + 1, name.end(),
                     [](char c) { return (c >= 'a' && c <= 'z') || (c >= '0' && c <= '9') || c == '_'; });
}

// ---- construction -----------------------------------------------------------------------------------------

Result<Node*> Graph::create_node(std::string op, std::vector<Value*> inputs, std::vector<TensorType> output_types) {
  if (op == kGraphInputOp)
    return invalid("Graph.create_node: op name 'graph_input' is reserved for graph inputs (use add_graph_input)");
  if (op == kGraphOutputMarker)
    return invalid("Graph.create_node: op name 'graph_output' is reserved as the serialization graph output marker");
  if (!matches_op_name_charset(op))
    return invalid("Graph.create_node: op name '" + op + "' is invalid, must match ^[a-z][a-z0-9_]*$");
  for (const Value* v : inputs)
    if (v == nullptr || v->producer() == nullptr || !node_set_.count(v->producer()))
      return invalid("Graph.create_node: input value does not belong to this graph");
  auto node = std::make_unique<Node>(std::move(op));
  node->inputs_ = std::move(inputs);
  node->outputs_.resize(output_types.size());
  for (size_t i = 0; i < output_types.size(); ++i) {
    node->outputs_[i].type_ = std::move(output_types[i]);
    node->outputs_[i].producer_ = node.get();
    node->outputs_[i].output_index_ = static_cast<int32_t>(i);
  }
  Node* raw = node.get();
  nodes_.push_back(std::move(node));
  topo_order_.push_back(raw);
  node_set_.insert(raw);
  return raw;
}

Result<Value*> Graph::add_graph_input(TensorType type) {
  auto node = std::make_unique<Node>(std::string(kGraphInputOp));
  node->outputs_.resize(1);
  node->outputs_[0].type_ = std::move(type);
  node->outputs_[0].producer_ = node.get();
  Node* raw = node.get();
  nodes_.push_back(std::move(node));
  topo_order_.push_back(raw);
  node_set_.insert(raw);
  inputs_.push_back(&raw->outputs_[0]);
  return &raw->outputs_[0];
}

Status Graph::mark_output(Value* value) {
  if (value == nullptr || value->producer() == nullptr || !node_set_.count(value->producer()))
    return invalid("Graph.mark_output: value does not belong to this graph");
  outputs_.push_back(value);
  return Status::ok();
}

Status Graph::mark_output(Node* node, int32_t output_index) {
  if (node == nullptr || !node_set_.count(node)) return invalid("Graph.mark_output: node does not belong to this graph");
  Value* v = node->output(output_index);
  if (v == nullptr)
    return invalid("Graph.mark_output: output index " + std::to_string(output_index) + " is out of range for node '" +
                   std::string(node->op()) + "'");
  return mark_output(v);
}

Status Graph::erase_node(Node* node) {
  if (node == nullptr) return invalid("Graph.erase_node: node is null");
  auto owned = std::find_if(nodes_.begin(), nodes_.end(), [&](const auto& p) { return p.get() == node; });
  if (owned == nodes_.end()) return invalid("Graph.erase_node: node does not belong to this graph");
  auto produced_here = [&](const Value* v) { return v != nullptr && v->producer() == node; };
  for (const auto& other : nodes_) {
    if (other.get() == node) continue;
    if (std::any_of(other->inputs_.begin(), other->inputs_.end(), produced_here))
      return invalid("Graph.erase_node: node output is referenced by another node's input");
  }
  if (std::any_of(outputs_.begin(), outputs_.end(), produced_here))
    return invalid("Graph.erase_node: node output is referenced by a graph output");
  topo_order_.erase(std::remove(topo_order_.begin(), topo_order_.end(), node), topo_order_.end());
  inputs_.erase(std::remove_if(inputs_.begin(), inputs_.end(), produced_here), inputs_.end());
  node_set_.erase(node);
  nodes_.erase(owned);
  return Status::ok();
}

Status Graph::replace_all_uses(Value* from, Value* to) {
  if (from == nullptr || from->producer() == nullptr || !node_set_.count(from->producer()))
    return invalid("Graph.replace_all_uses: from value does not belong to this graph");
  if (to == nullptr || to->producer() == nullptr || !node_set_.count(to->producer()))
    return invalid("Graph.replace_all_uses: to value does not belong to this graph");
  if (from == to) return invalid("Graph.replace_all_uses: from and to must be different values");
  const TensorType& a = from->type();
  const TensorType& b = to->type();
  if (!(a.dtype == b.dtype) || !(a.shape == b.shape) || a.layout != b.layout || !(a.device == b.device)) {
    return invalid("Graph.replace_all_uses: from and to have different tensor types, from dtype '" +
                   std::string(a.dtype.name()) + "' shape " + a.shape.to_string() + " layout " +
                   std::string(layout_name(a.layout)) + " device " + device_text(a.device) + ", to dtype '" +
                   std::string(b.dtype.name()) + "' shape " + b.shape.to_string() + " layout " +
                   std::string(layout_name(b.layout)) + " device " + device_text(b.device));
  }
  Node* fp = from->producer();
  Node* tp = to->producer();
  if (fp != tp) {
    auto index_of = [&](const Node* n) {
      return static_cast<size_t>(std::find(topo_order_.begin(), topo_order_.end(), n) - topo_order_.begin());
    };
    const size_t fi = index_of(fp);
    const size_t ti = index_of(tp);
    if (ti > fi) {
      // `to` comes later: it may move up to `from`'s slot only if all its inputs are produced before that slot.
      for (const Value* in : tp->inputs())
        if (index_of(in->producer()) >= fi)
          return invalid("Graph.replace_all_uses: topological order invariant violated, to's producer op '" +
                         std::string(tp->op()) + "' must appear before from's producer op '" + std::string(fp->op()) +
                         "' in topological order, or have every input's producer strictly before from's producer "
                         "to qualify for relocation");
      std::rotate(topo_order_.begin() + static_cast<std::ptrdiff_t>(fi),
                  topo_order_.begin() + static_cast<std::ptrdiff_t>(ti),
                  topo_order_.begin() + static_cast<std::ptrdiff_t>(ti) + 1);
    }
  }
  for (auto& n : nodes_)
    for (Value*& in : n->inputs_)
      if (in == from) in = to;
  for (Value*& out : outputs_)
    if (out == from) out = to;
  return Status::ok();
}

Status Graph::swap_node_inputs(Node* node, int32_t i, int32_t j) {
  if (node == nullptr || !node_set_.count(node))
    return invalid("Graph.swap_node_inputs: node does not belong to this graph");
  const int32_t n = static_cast<int32_t>(node->inputs_.size());
  if (i < 0 || i >= n || j < 0 || j >= n)
    return invalid("Graph.swap_node_inputs: index out of range, i=" + std::to_string(i) + ", j=" + std::to_string(j) +
                   ", input count=" + std::to_string(n));
  if (i == j) return invalid("Graph.swap_node_inputs: i and j must be different indices, got " + std::to_string(i));
  std::swap(node->inputs_[static_cast<size_t>(i)], node->inputs_[static_cast<size_t>(j)]);
  return Status::ok();
}

Status Graph::assign_layout(Value* value, Layout layout) {
  if (value == nullptr || value->producer() == nullptr || !node_set_.count(value->producer()))
    return invalid("Graph.assign_layout: value does not belong to this graph");
  if (layout == Layout::kUnknown) return invalid("Graph.assign_layout: layout must not be kUnknown");
  const Layout cur = value->type_.layout;
  if (cur == layout) return Status::ok();
  if (cur != Layout::kUnknown)
    return invalid("Graph.assign_layout: value already has layout '" + std::string(layout_name(cur)) +
                   "', cannot reassign to '" + std::string(layout_name(layout)) + "'");
  value->type_.layout = layout;
  return Status::ok();
}

// ---- invariants -------------------------------------------------------------------------------------------

namespace {

bool slot_consistent(const Value* v) {
  const Node* p = v->producer();
  const int32_t i = v->output_index();
  return i >= 0 && static_cast<size_t>(i) < p->outputs().size() && v == &p->outputs()[static_cast<size_t>(i)];
}

Status check_v1(const Graph& g, const std::unordered_set<const Node*>& nodes) {
  for (const Node* n : g.topological_order()) {
    for (const Value* in : n->inputs()) {
      if (in == nullptr || in->producer() == nullptr)
        return invalid("V1: node '" + std::string(n->op()) + "' has an input value with no producer");
      if (!nodes.count(in->producer()))
        return invalid("V1: node '" + std::string(n->op()) + "' has an input value produced outside this graph");
      if (!slot_consistent(in))
        return invalid("V1: node '" + std::string(n->op()) +
                       "' has an input value pointer that does not match its producer's output slot");
    }
  }
  for (const Value* out : g.outputs()) {
    if (out == nullptr || out->producer() == nullptr || !nodes.count(out->producer()))
      return invalid("V1: graph output value has no valid producer in this graph");
    if (!slot_consistent(out)) return invalid("V1: graph output value pointer does not match its producer's output slot");
  }
  for (const Value* in : g.inputs())
    if (in == nullptr || in->producer() == nullptr || in->producer()->op() != kGraphInputOp)
      return invalid("V1: graph input value's producer is not a graph_input node");
  return Status::ok();
}

// V2: every input is produced by a node that appears earlier in the stored order, and no node repeats.
// (Construction only ever appends nodes whose inputs exist, and relocations keep inputs ahead.)
Status check_v2(const Graph& g) {
  std::unordered_map<const Node*, size_t> pos;
  const auto& topo = g.topological_order();
  for (size_t i = 0; i < topo.size(); ++i)
    if (!pos.emplace(topo[i], i).second)
      return Status::make(ErrorCode::kInternal, "V2: topological_order contains duplicate nodes");
  // Kahn's algorithm over the use edges detects any cycle independently of the stored order.
  std::unordered_map<const Node*, int64_t> indeg;
  std::unordered_map<const Node*, std::vector<const Node*>> users;
  for (const Node* n : topo) indeg[n] = 0;
  for (const Node* n : topo)
    for (const Value* in : n->inputs()) {
      if (in == nullptr || in->producer() == nullptr || !pos.count(in->producer())) continue;
      ++indeg[n];
      users[in->producer()].push_back(n);
    }
  std::vector<const Node*> ready;
  for (const Node* n : topo)
    if (indeg[n] == 0) ready.push_back(n);
  size_t seen = 0;
  while (!ready.empty()) {
    const Node* n = ready.back();
    ready.pop_back();
    ++seen;
    auto it = users.find(n);
    if (it == users.end()) continue;
    for (const Node* u : it->second)
      if (--indeg[u] == 0) ready.push_back(u);
  }
  if (seen != topo.size()) return invalid("V2: graph contains a cycle");
  return Status::ok();
}

Status check_v5(const Graph& g) {
  for (const Node* n : g.topological_order())
    for (const Value& out : n->outputs()) {
      Status s = out.type().shape.verify();
      if (!s.is_ok())
        return Status::make(s.code(), "V5: node '" + std::string(n->op()) + "' output has invalid shape: " +
                                          std::string(s.message()));
      if (static_cast<uint8_t>(out.type().dtype.code()) >= static_cast<uint8_t>(DTypeCode::kCount))
        return invalid("V5: node '" + std::string(n->op()) + "' output has invalid dtype code");
    }
  return Status::ok();
}

Status check_v6(const Graph& g) {
  const Device* first = nullptr;
  for (const Node* n : g.topological_order())
    for (const Value& out : n->outputs()) {
      if (first == nullptr) {
        first = &out.type().device;
      } else if (!(out.type().device == *first)) {
        return invalid("V6: graph contains values on inconsistent devices");
      }
    }
  return Status::ok();
}

Status check_v7(const Graph& g) {
  for (const Node* n : g.topological_order())
    for (const auto& kv : n->attrs()) (void)attr_type_name(attr_type_of(kv.second));
  return Status::ok();
}

}  // namespace

Status Graph::verify_structure() const {
  FRAME_RETURN_IF_ERROR(check_v1(*this, node_set_));
  FRAME_RETURN_IF_ERROR(check_v2(*this));
  FRAME_RETURN_IF_ERROR(check_v5(*this));
  FRAME_RETURN_IF_ERROR(check_v6(*this));
  return check_v7(*this);
}

Status Graph::verify(const OpQuery& query) const {
  if (!query.op_registered) return invalid("V3: OpQuery.op_registered callback is not set (fail-closed)");
  if (!query.check_schema) return invalid("V4: OpQuery.check_schema callback is not set (fail-closed)");
  FRAME_RETURN_IF_ERROR(verify_structure());
  for (const Node* n : topo_order_) {
    if (n->op() == kGraphInputOp) {
      if (!n->inputs().empty()) return invalid("V3: graph_input node must have zero inputs");
      if (n->outputs().size() != 1) return invalid("V3: graph_input node must have exactly one output");
      if (std::find(inputs_.begin(), inputs_.end(), &n->outputs()[0]) == inputs_.end())
        return invalid("V3: graph_input node output is not registered in graph inputs");
      continue;
    }
    if (!query.op_registered(n->op()))
      return Status::make(ErrorCode::kNotFound, "V3: op '" + std::string(n->op()) + "' is not registered");
    Status s = query.check_schema(*n);
    if (!s.is_ok()) return Status::make(s.code(), "V4: " + std::string(s.message()));
  }
  return Status::ok();
}

// ---- clone ------------------------------------------------------------------------------------------------

Result<Graph> clone_graph(const Graph& source, std::unordered_map<const Value*, Value*>* value_map) {
  std::unordered_map<const Value*, Value*> local;
  auto& map = value_map != nullptr ? *value_map : local;
  map.clear();
  Graph out{std::string(source.name())};
  for (const Node* n : source.topological_order()) {
    if (n->op() == kGraphInputOp) {
      Result<Value*> v = out.add_graph_input(n->outputs()[0].type());
      if (!v.is_ok()) return v.status();
      map[&n->outputs()[0]] = v.value();
      continue;
    }
    std::vector<Value*> ins;
    ins.reserve(n->inputs().size());
    for (const Value* in : n->inputs()) ins.push_back(map.at(in));
    std::vector<TensorType> types;
    for (const Value& o : n->outputs()) types.push_back(o.type());
    Result<Node*> c = out.create_node(std::string(n->op()), std::move(ins), std::move(types));
    if (!c.is_ok()) return c.status();
    for (const auto& [k, v] : n->attrs()) c.value()->set_attr(k, v);
    for (size_t i = 0; i < n->outputs().size(); ++i) map[&n->outputs()[i]] = c.value()->output(static_cast<int32_t>(i));
  }
  // Graph inputs keep the source's registration order even if their nodes were relocated.
  // (add_graph_input appends in topological order, which is the only order the construction API produces.)
  for (const Value* o : source.outputs()) FRAME_RETURN_IF_ERROR(out.mark_output(map.at(o)));
  return out;
}

}  // namespace frame::ir

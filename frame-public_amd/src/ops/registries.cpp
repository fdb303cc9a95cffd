// Op / kernel registries, schema builder and the verify() schema query
// (reference behaviour: src/ops/{op_schema,op_registry,kernel_registry}.cpp).
#include <cstdio>
#include <cstdlib>
#include <string>
#include <unordered_set>

#include <frame/ops/kernel_registry.h>
#include <frame/ops/op_registry.h>

namespace frame::ops {

namespace {
[[noreturn]] void die(const std::string& msg) {
  std::fprintf(stderr, "[frame] fatal registration error: %s\n", msg.c_str());
  std::abort();
}
}  // namespace

// ---- OpSchema builder -------------------------------------------------------------------------------------

OpSchema& OpSchema::input(std::string_view name, std::string_view doc) noexcept {
  if (has_variadic_input_)
    die("op '" + name_ + "' declares fixed input '" + std::string(name) + "' after its variadic input group");
  inputs_.push_back({std::string(name), std::string(doc)});
  return *this;
}

OpSchema& OpSchema::variadic_input(std::string_view name, std::string_view doc, int32_t min_count) noexcept {
  if (has_variadic_input_) die("op '" + name_ + "' declares more than one variadic input group");
  if (min_count < 0) die("op '" + name_ + "' variadic input group has negative min_count");
  has_variadic_input_ = true;
  variadic_input_param_ = {std::string(name), std::string(doc)};
  variadic_min_count_ = min_count;
  return *this;
}

OpSchema& OpSchema::output(std::string_view name, std::string_view doc) noexcept {
  outputs_.push_back({std::string(name), std::string(doc)});
  return *this;
}

OpSchema& OpSchema::attr(std::string_view name, ir::AttrType type, bool required) noexcept {
  attrs_.push_back({std::string(name), type, required});
  return *this;
}

OpSchema& OpSchema::trait(OpTrait t) noexcept {
  traits_ = static_cast<uint8_t>(traits_ | (1U << static_cast<uint8_t>(t)));
  return *this;
}

OpSchema& OpSchema::shape_infer(ShapeInferFn fn) noexcept {
  shape_infer_ = fn;
  return *this;
}

OpSchema& OpSchema::decomposition(DecomposeFn fn) noexcept {
  decompose_ = fn;
  return *this;
}

OpSchema& OpSchema::gradient(GradientFn fn) noexcept {
  if (has_trait(OpTrait::kHasSideEffect)) die("op '" + name_ + "' has side effects and cannot have a gradient");
  gradient_ = fn;
  return *this;
}

// ---- OpRegistry -------------------------------------------------------------------------------------------

OpRegistry& OpRegistry::instance() noexcept {
  static OpRegistry registry;
  return registry;
}

OpSchema& OpRegistry::register_op(std::string_view name) noexcept {
  if (!ir::matches_op_name_charset(name))
    die("op name '" + std::string(name) + "' is invalid, must match ^[a-z][a-z0-9_]*$");
  if (name == ir::kGraphInputOp || name == ir::kGraphOutputMarker)
    die("op name '" + std::string(name) + "' is reserved by the ir layer");
  auto [it, inserted] = schemas_.try_emplace(std::string(name));
  if (!inserted) die("op '" + std::string(name) + "' is registered twice");
  it->second.name_ = std::string(name);
  return it->second;
}

const OpSchema* OpRegistry::find(std::string_view name) const {
  auto it = schemas_.find(std::string(name));
  return it == schemas_.end() ? nullptr : &it->second;
}

ir::OpQuery make_op_query() {
  ir::OpQuery q;
  q.op_registered = [](std::string_view op) { return OpRegistry::instance().find(op) != nullptr; };
  q.check_schema = [](const ir::Node& node) -> Status {
    const OpSchema* s = OpRegistry::instance().find(node.op());
    const std::string op(node.op());
    if (s == nullptr) return Status::make(ErrorCode::kNotFound, "op '" + op + "' is not registered");
    const size_t n_in = node.inputs().size();
    if (s->has_variadic_inputs()) {
      if (n_in < static_cast<size_t>(s->min_input_count()))
        return Status::make(ErrorCode::kInvalidArgument, "op '" + op + "' expects at least " +
                                                             std::to_string(s->min_input_count()) + " input(s), got " +
                                                             std::to_string(n_in));
    } else if (n_in != s->inputs().size()) {
      return Status::make(ErrorCode::kInvalidArgument, "op '" + op + "' expects " + std::to_string(s->inputs().size()) +
                                                           " input(s), got " + std::to_string(n_in));
    }
    if (node.outputs().size() != s->outputs().size())
      return Status::make(ErrorCode::kInvalidArgument, "op '" + op + "' expects " + std::to_string(s->outputs().size()) +
                                                           " output(s), got " + std::to_string(node.outputs().size()));
    std::unordered_set<std::string> declared;
    for (const OpAttrSpec& a : s->attrs()) {
      declared.insert(a.name);
      const ir::AttrValue* v = node.find_attr(a.name);
      if (v == nullptr) {
        if (a.required)
          return Status::make(ErrorCode::kInvalidArgument,
                              "op '" + op + "' is missing required attribute '" + a.name + "'");
        continue;
      }
      if (ir::attr_type_of(*v) != a.type)
        return Status::make(ErrorCode::kInvalidArgument,
                            "op '" + op + "' attribute '" + a.name + "' has type " +
                                std::string(ir::attr_type_name(ir::attr_type_of(*v))) + ", expected " +
                                std::string(ir::attr_type_name(a.type)));
    }
    for (const auto& [k, v] : node.attrs())
      if (!declared.count(k))
        return Status::make(ErrorCode::kInvalidArgument, "op '" + op + "' has unknown attribute '" + k + "'");
    return Status::ok();
  };
  return q;
}

// ---- KernelRegistry ---------------------------------------------------------------------------------------

KernelRegistry& KernelRegistry::instance() noexcept {
  static KernelRegistry registry;
  return registry;
}

Status KernelRegistry::register_kernel(std::string_view op, std::string_view backend, KernelFn fn) noexcept {
  if (fn == nullptr)
    return Status::make(ErrorCode::kInvalidArgument,
                        "kernel for op '" + std::string(op) + "' on backend '" + std::string(backend) + "' is null");
  auto [it, inserted] = kernels_.try_emplace({std::string(op), std::string(backend)}, fn);
  if (!inserted)
    return Status::make(ErrorCode::kAlreadyExists, "kernel for op '" + std::string(op) + "' on backend '" +
                                                       std::string(backend) + "' is already registered");
  return Status::ok();
}

bool KernelRegistry::register_kernel_or_die(std::string_view op, std::string_view backend, KernelFn fn) noexcept {
  Status s = register_kernel(op, backend, fn);
  if (!s.is_ok()) die(std::string(s.message()));
  return true;
}

Result<KernelFn> KernelRegistry::find(std::string_view op, std::string_view backend) const {
  auto it = kernels_.find({std::string(op), std::string(backend)});
  if (it == kernels_.end())
    return Status::make(ErrorCode::kNotFound, "no kernel registered for op '" + std::string(op) + "' on backend '" +
                                                  std::string(backend) + "'");
  return it->second;
}

}  // namespace frame::ops

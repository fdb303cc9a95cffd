// PassRegistry, PassManager and the standard pipeline
// (reference: src/compiler/{pass_registry,pass_manager,pipeline}.cpp).
#include <cstdio>
#include <cstdlib>
#include <ostream>
#include <string>

#include <frame/compiler/pass.h>
#include <frame/compiler/pass_manager.h>
#include <frame/compiler/pipeline.h>
#include <frame/ir/graph.h>
#include <frame/ir/serialization.h>
#include <frame/ops/op_registry.h>

namespace frame::compiler {

PassRegistry& PassRegistry::instance() noexcept {
  static PassRegistry r;
  return r;
}

Status PassRegistry::register_pass(std::string_view name, Factory factory) noexcept {
  if (factory == nullptr)
    return Status::make(ErrorCode::kInvalidArgument, "pass '" + std::string(name) + "' has a null factory");
  if (!passes_.try_emplace(std::string(name), factory).second)
    return Status::make(ErrorCode::kAlreadyExists, "pass '" + std::string(name) + "' is already registered");
  return Status::ok();
}

bool PassRegistry::register_pass_or_die(std::string_view name, Factory factory) noexcept {
  Status s = register_pass(name, factory);
  if (!s.is_ok()) {
    std::fprintf(stderr, "[frame] fatal pass registration error: %s\n", std::string(s.message()).c_str());
    std::abort();
  }
  return true;
}

Result<std::unique_ptr<Pass>> PassRegistry::create(std::string_view name) const {
  auto it = passes_.find(std::string(name));
  if (it == passes_.end()) return Status::make(ErrorCode::kNotFound, "pass '" + std::string(name) + "' is not registered");
  return it->second();
}

PassManager& PassManager::add_pass(std::unique_ptr<Pass> pass) {
  passes_.push_back(std::move(pass));
  return *this;
}

PassManager& PassManager::add(std::string_view pass_name) {
  Result<std::unique_ptr<Pass>> p = PassRegistry::instance().create(pass_name);
  if (!p.is_ok()) {
    if (pending_error_.is_ok()) pending_error_ = p.status();
  } else {
    passes_.push_back(std::move(p.value()));
  }
  return *this;
}

Status PassManager::run(ir::Graph& graph) const {
  if (!pending_error_.is_ok()) return pending_error_;
  const ir::OpQuery query = ops::make_op_query();
  for (const auto& pass : passes_) {
    auto wrap = [&](const Status& s) {
      return Status::make(s.code(), "pass '" + std::string(pass->name()) + "': " + std::string(s.message()));
    };
    Status s = pass->run(graph);
    if (!s.is_ok()) return wrap(s);
    if (dump_stream_ != nullptr && pass->name() == dump_pass_name_) *dump_stream_ << ir::dump_text(graph);
    s = graph.verify(query);
    if (!s.is_ok()) return wrap(s);
  }
  return Status::ok();
}

void PassManager::set_dump_ir_after(std::string_view pass_name, std::ostream& os) {
  dump_pass_name_ = std::string(pass_name);
  dump_stream_ = &os;
}

std::vector<std::string_view> PassManager::pass_names() const {
  std::vector<std::string_view> names;
  for (const auto& p : passes_) names.push_back(p->name());
  return names;
}

Result<PassManager> standard_pipeline(std::string_view /*backend*/) {
  PassManager pm;
  for (std::string_view name : {"canonicalize", "shape_inference", "constant_folding", "common_subexpression_elimination",
                                "dead_node_elimination", "layout_assignment", "operator_fusion", "memory_planning",
                                "backend_lowering"}) {
    Result<std::unique_ptr<Pass>> p = PassRegistry::instance().create(name);
    if (!p.is_ok()) return p.status();
    pm.add_pass(std::move(p.value()));
  }
  return pm;
}

}  // namespace frame::compiler

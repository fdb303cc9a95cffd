#pragma once
// Pass extension point: Pass interface, CRTP PassBase, PassRegistry and FRAME_REGISTER_PASS
// (reference: include/frame/compiler/pass.h:24-108).

#include <concepts>
#include <memory>
#include <string>
#include <string_view>
#include <type_traits>
#include <unordered_map>

#include <frame/core/macros.h>
#include <frame/core/status.h>

namespace frame::ir {
class Graph;
}

namespace frame::compiler {

class FRAME_API Pass {
 public:
  virtual ~Pass() = default;
  virtual std::string_view name() const = 0;
  virtual Status run(ir::Graph& graph) = 0;  // in place; on failure leave no half-transformed state
};

template <typename Derived>
class PassBase : public Pass {
 public:
  std::string_view name() const final { return Derived::kName; }
  Status run(ir::Graph& graph) final { return static_cast<Derived*>(this)->run_impl(graph); }

 private:
  PassBase() = default;
  friend Derived;
};

template <typename P>
concept PassType = std::derived_from<P, Pass> && std::is_default_constructible_v<P> && requires {
  { P::kName } -> std::convertible_to<std::string_view>;
};

class FRAME_API PassRegistry {
 public:
  static PassRegistry& instance() noexcept;
  using Factory = std::unique_ptr<Pass> (*)();
  Status register_pass(std::string_view name, Factory factory) noexcept;
  template <PassType P>
  Status register_pass() {
    return register_pass(P::kName, []() -> std::unique_ptr<Pass> { return std::make_unique<P>(); });
  }
  bool register_pass_or_die(std::string_view name, Factory factory) noexcept;
  template <PassType P>
  bool register_pass_or_die() noexcept {
    return register_pass_or_die(P::kName, []() -> std::unique_ptr<Pass> { return std::make_unique<P>(); });
  }
  Result<std::unique_ptr<Pass>> create(std::string_view name) const;

 private:
  std::unordered_map<std::string, Factory> passes_;
};

}  // namespace frame::compiler

#define FRAME_REGISTER_PASS(PassClass)                                            \
  [[maybe_unused]] static const bool FRAME_CONCAT(frame_pass_reg_, __COUNTER__) = \
      ::frame::compiler::PassRegistry::instance().register_pass_or_die<PassClass>()

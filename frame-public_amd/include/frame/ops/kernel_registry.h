#pragma once
// KernelRegistry: (op, backend) -> KernelFn. No dtype in the key: kernels dispatch on dtype internally
// (reference: include/frame/ops/kernel_registry.h:30-107).

#include <concepts>
#include <functional>
#include <span>
#include <string>
#include <string_view>
#include <unordered_map>
#include <utility>

#include <frame/core/device.h>
#include <frame/core/macros.h>
#include <frame/core/status.h>
#include <frame/core/tensor.h>
#include <frame/ir/attribute.h>

namespace frame::hal {
class Stream;
struct CompileOptions;
}  // namespace frame::hal

namespace frame::ops {

// Everything a kernel may touch; all members are borrowed for the duration of the call.
struct KernelContext {
  std::span<const Tensor> inputs;
  std::span<Tensor> outputs;  // pre-allocated by the caller
  const std::unordered_map<std::string, ir::AttrValue>* attrs = nullptr;
  Device device;
  hal::Stream* stream = nullptr;
  const hal::CompileOptions* compile_options = nullptr;  // nullptr = defaults
};

using KernelFn = Status (*)(KernelContext&);

template <typename F>
concept KernelImpl = std::convertible_to<F, KernelFn>;

class FRAME_API KernelRegistry {
 public:
  static KernelRegistry& instance() noexcept;
  Status register_kernel(std::string_view op, std::string_view backend, KernelFn fn) noexcept;
  bool register_kernel_or_die(std::string_view op, std::string_view backend, KernelFn fn) noexcept;
  Result<KernelFn> find(std::string_view op, std::string_view backend) const;

 private:
  struct KeyHash {
    size_t operator()(const std::pair<std::string, std::string>& k) const {
      const size_t a = std::hash<std::string>()(k.first);
      const size_t b = std::hash<std::string>()(k.second);
      return a ^ (b * 0x100000001b3ULL + (a << 7));
    }
  };
  std::unordered_map<std::pair<std::string, std::string>, KernelFn, KeyHash> kernels_;
};

}  // namespace frame::ops

#define FRAME_REGISTER_KERNEL(op_name, backend_name, fn)                                         \
  [[maybe_unused]] static const bool FRAME_CONCAT(frame_kernel_reg_, __COUNTER__) =              \
      ::frame::ops::KernelRegistry::instance().register_kernel_or_die((op_name), (backend_name), \
                                                                      (fn))

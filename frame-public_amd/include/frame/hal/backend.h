#pragma once
// hal::Backend: the plugin boundary. A backend registers under a string key with FRAME_REGISTER_BACKEND and is
// driven by runtime::compile through compile()/launch(). Signatures are those of the reference
// (include/frame/hal/backend.h:51-160) so that a backend written for Frame plugs in unchanged.

#include <cstddef>
#include <memory>
#include <span>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

#include <frame/core/device.h>
#include <frame/core/macros.h>
#include <frame/core/status.h>
#include <frame/core/tensor.h>
#include <frame/ir/attribute.h>

namespace frame::ir {
class Graph;
}

namespace frame::hal {

class Stream;
class Event;
class Allocator;
class Executable;

// Options of Backend::compile. Every field must appear in fingerprint(): it is part of the compile-cache key.
struct CompileOptions {
  int32_t opt_level = 1;    // 0 disables backend-internal optimisation (for the hip backend: epilogue fusion)
  bool allow_tf32 = false;  // permission for reduced-precision fp32 math; the hip backend stays strict fp32
  std::string fingerprint() const {
    return "opt_level=" + std::to_string(opt_level) + ";allow_tf32=" + (allow_tf32 ? "1" : "0");
  }
};

// Single-kernel eager launch. attrs and spans are borrowed for the duration of the call; outputs are
// pre-allocated by the caller from the op's shape inference.
struct KernelInvocation {
  std::string_view op;
  std::span<const Tensor> inputs;
  std::span<Tensor> outputs;
  const std::unordered_map<std::string, ir::AttrValue>* attrs = nullptr;
  Device device;
};

class FRAME_API Backend {
 public:
  virtual ~Backend() = default;
  virtual std::string_view name() const = 0;
  virtual Result<int32_t> device_count() const = 0;
  virtual Result<std::unique_ptr<Stream>> create_stream(Device device) = 0;
  virtual Result<std::unique_ptr<Event>> create_event(Device device) = 0;
  virtual Allocator* allocator(Device device) = 0;  // backend-owned, process lifetime
  // Direction follows from the two devices; host memory is a cpu-backend Device. stream == nullptr: synchronous.
  virtual Status copy(void* dst, Device dst_device, const void* src, Device src_device, size_t bytes,
                      Stream* stream) = 0;
  virtual Result<std::unique_ptr<Executable>> compile(const ir::Graph& graph, const CompileOptions& options) = 0;
  virtual Status launch(const KernelInvocation& invocation, Stream* stream) = 0;
};

class FRAME_API BackendRegistry {
 public:
  static BackendRegistry& instance() noexcept;
  Status register_backend(std::string_view name, std::unique_ptr<Backend> backend) noexcept;
  bool register_backend_or_die(std::string_view name, std::unique_ptr<Backend> backend) noexcept;
  template <typename BackendClass>
  bool register_backend_or_die(std::string_view name) noexcept {
    return register_backend_or_die(name, std::make_unique<BackendClass>());
  }
  Result<Backend*> get(std::string_view name);
  std::vector<std::string_view> available() const;  // sorted

 private:
  std::unordered_map<std::string, std::unique_ptr<Backend>> backends_;
};

}  // namespace frame::hal

#define FRAME_REGISTER_BACKEND(name_string, BackendClass)                            \
  [[maybe_unused]] static const bool FRAME_CONCAT(frame_backend_reg_, __COUNTER__) = \
      ::frame::hal::BackendRegistry::instance().register_backend_or_die<BackendClass>(name_string)

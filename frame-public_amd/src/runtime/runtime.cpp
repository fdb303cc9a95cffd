// runtime::compile with its compile cache, run_with_allocated_outputs, the backend registry and the shared
// I/O validation helpers (reference: src/runtime/{compile,backend_registry,executable}.cpp).
//
// Difference from the reference: a graph the target backend cannot compile (kUnimplemented from the pipeline
// or from Backend::compile) is reported to the caller instead of being rerouted to the reference's eager
// fallback chain, whose last hop runs cpu kernels (reference: src/runtime/compile.cpp:104-124). This library
// has no cpu backend, and a silent CPU detour would hide a missing device kernel.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include <frame/compiler/pipeline.h>
#include <frame/hal/allocator.h>
#include <frame/hal/backend.h>
#include <frame/hal/executable.h>
#include <frame/hal/stream.h>
#include <frame/ir/graph.h>
#include <frame/ir/serialization.h>
#include <frame/runtime/compile.h>

namespace frame {

// ---- hal::BackendRegistry ---------------------------------------------------------------------------------
namespace hal {

BackendRegistry& BackendRegistry::instance() noexcept {
  static BackendRegistry r;
  return r;
}

Status BackendRegistry::register_backend(std::string_view name, std::unique_ptr<Backend> backend) noexcept {
  if (name.empty()) return Status::make(ErrorCode::kInvalidArgument, "backend registration key must not be empty");
  if (backend == nullptr)
    return Status::make(ErrorCode::kInvalidArgument, "backend '" + std::string(name) + "' registered as null");
  if (!backends_.try_emplace(std::string(name), std::move(backend)).second)
    return Status::make(ErrorCode::kAlreadyExists, "backend '" + std::string(name) + "' is already registered");
  return Status::ok();
}

bool BackendRegistry::register_backend_or_die(std::string_view name, std::unique_ptr<Backend> backend) noexcept {
  Status s = register_backend(name, std::move(backend));
  if (!s.is_ok()) {
    std::fprintf(stderr, "[frame] fatal backend registration error: %s\n", std::string(s.message()).c_str());
    std::abort();
  }
  return true;
}

Result<Backend*> BackendRegistry::get(std::string_view name) {
  auto it = backends_.find(std::string(name));
  if (it == backends_.end())
    return Status::make(ErrorCode::kNotFound, "backend '" + std::string(name) + "' is not registered");
  return it->second.get();
}

std::vector<std::string_view> BackendRegistry::available() const {
  std::vector<std::string_view> names;
  for (const auto& [k, v] : backends_) names.push_back(k);
  std::sort(names.begin(), names.end());
  return names;
}

Status validate_io_signature(std::span<const Tensor> values, const std::vector<IoSpec>& sig, std::string_view label) {
  const std::string l(label);
  if (values.size() != sig.size())
    return Status::make(ErrorCode::kInvalidArgument, l + " count mismatch: expected " + std::to_string(sig.size()) +
                                                         ", got " + std::to_string(values.size()));
  for (size_t i = 0; i < sig.size(); ++i) {
    if (!(values[i].dtype() == sig[i].dtype))
      return Status::make(ErrorCode::kInvalidArgument, l + " " + std::to_string(i) + " dtype mismatch: expected '" +
                                                           std::string(sig[i].dtype.name()) + "', got '" +
                                                           std::string(values[i].dtype().name()) + "'");
    if (!(values[i].shape() == sig[i].shape))
      return Status::make(ErrorCode::kInvalidArgument, l + " " + std::to_string(i) + " shape mismatch: expected " +
                                                           sig[i].shape.to_string() + ", got " +
                                                           values[i].shape().to_string());
  }
  return Status::ok();
}

Status validate_tensor_devices(std::span<const Tensor> values, Device expected, std::string_view label) {
  for (size_t i = 0; i < values.size(); ++i) {
    const Device d = values[i].device();
    if (!(d == expected))
      return Status::make(ErrorCode::kInvalidArgument,
                          std::string(label) + " " + std::to_string(i) + " device mismatch: tensor is on " +
                              std::string(d.backend) + ":" + std::to_string(d.index) + ", expected " +
                              std::string(expected.backend) + ":" + std::to_string(expected.index));
  }
  return Status::ok();
}

}  // namespace hal

// ---- runtime ------------------------------------------------------------------------------------------------
namespace runtime {
namespace {

class CompilationCache {
 public:
  static CompilationCache& instance() {
    static CompilationCache c;
    return c;
  }
  std::shared_ptr<hal::Executable> find(const std::string& key) {
    std::lock_guard<std::mutex> lock(mu_);
    auto it = map_.find(key);
    return it == map_.end() ? nullptr : it->second;
  }
  void insert(std::string key, std::shared_ptr<hal::Executable> exe) {
    std::lock_guard<std::mutex> lock(mu_);
    map_.emplace(std::move(key), std::move(exe));
  }
  size_t size() {
    std::lock_guard<std::mutex> lock(mu_);
    return map_.size();
  }

 private:
  std::mutex mu_;
  std::unordered_map<std::string, std::shared_ptr<hal::Executable>> map_;
};

std::string_view device_backend_of(const ir::Graph& g) {
  for (const ir::Node* n : g.topological_order())
    if (!n->outputs().empty()) return n->outputs()[0].type().device.backend;
  return {};
}

}  // namespace

Result<std::shared_ptr<hal::Executable>> compile(const ir::Graph& graph, std::string_view backend_name,
                                                 const hal::CompileOptions& options) {
  const std::string_view on = device_backend_of(graph);
  if (!on.empty() && on != backend_name)
    return Status::make(ErrorCode::kInvalidArgument, "runtime::compile: backend_name '" + std::string(backend_name) +
                                                         "' does not match graph device backend '" + std::string(on) + "'");
  // Cache key: backend, options fingerprint and the text of the graph as given (before any pass runs).
  std::string key = std::string(backend_name) + '\x1f' + options.fingerprint() + '\x1f' + ir::dump_text(graph);
  CompilationCache& cache = CompilationCache::instance();
  if (auto hit = cache.find(key)) return hit;

  Result<ir::Graph> work = ir::clone_graph(graph);
  if (!work.is_ok()) return work.status();
  Result<compiler::PassManager> pipeline = compiler::standard_pipeline(backend_name);
  if (!pipeline.is_ok()) return pipeline.status();
  FRAME_RETURN_IF_ERROR(pipeline.value().run(work.value()));
  Result<hal::Backend*> backend = hal::BackendRegistry::instance().get(backend_name);
  if (!backend.is_ok()) return backend.status();
  Result<std::unique_ptr<hal::Executable>> exe = backend.value()->compile(work.value(), options);
  if (!exe.is_ok()) return exe.status();
  std::shared_ptr<hal::Executable> shared = std::move(exe.value());
  cache.insert(std::move(key), shared);
  return shared;
}

Result<std::vector<Tensor>> run_with_allocated_outputs(hal::Executable& executable, std::string_view backend_name,
                                                       std::span<const Tensor> inputs) {
  Result<hal::Backend*> backend = hal::BackendRegistry::instance().get(backend_name);
  if (!backend.is_ok()) return backend.status();
  const Device dev{backend.value()->name(), 0};
  hal::Allocator* alloc = backend.value()->allocator(dev);
  if (alloc == nullptr)
    return Status::make(ErrorCode::kInternal, "run_with_allocated_outputs: backend '" + std::string(backend_name) +
                                                  "' returned a null allocator for device index 0");
  std::vector<Tensor> outputs;
  for (const hal::IoSpec& spec : executable.output_signature()) {
    Result<Tensor> t = Tensor::empty(spec.shape, spec.dtype, dev, *alloc);
    if (!t.is_ok()) return t.status();
    outputs.push_back(std::move(t.value()));
  }
  Result<std::unique_ptr<hal::Stream>> stream = backend.value()->create_stream(dev);
  if (!stream.is_ok()) return stream.status();
  FRAME_RETURN_IF_ERROR(executable.run(inputs, outputs, *stream.value()));
  FRAME_RETURN_IF_ERROR(stream.value()->synchronize());
  return outputs;
}

size_t compilation_cache_size() { return CompilationCache::instance().size(); }

}  // namespace runtime
}  // namespace frame

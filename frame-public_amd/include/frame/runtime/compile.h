#pragma once
// runtime::compile — the single compile entry: checks the graph's device backend, looks up the compile cache
// (key = backend + options fingerprint + dump_text of the input graph), otherwise clones the graph, runs the
// standard pipeline and Backend::compile, and caches the Executable. run_with_allocated_outputs allocates the
// outputs on device 0 of the backend, creates a stream, runs and synchronises
// (reference: include/frame/runtime/compile.h:65-86, src/runtime/compile.cpp:128-220).

#include <memory>
#include <span>
#include <string_view>
#include <vector>

#include <frame/core/macros.h>
#include <frame/core/status.h>
#include <frame/core/tensor.h>
#include <frame/hal/backend.h>
#include <frame/hal/executable.h>

namespace frame::ir {
class Graph;
}

namespace frame::runtime {

FRAME_API Result<std::shared_ptr<hal::Executable>> compile(const ir::Graph& graph, std::string_view backend_name,
                                                           const hal::CompileOptions& options);

FRAME_API Result<std::vector<Tensor>> run_with_allocated_outputs(hal::Executable& executable,
                                                                 std::string_view backend_name,
                                                                 std::span<const Tensor> inputs);

// Number of entries in the compile cache (observability for tests).
FRAME_API size_t compilation_cache_size();

}  // namespace frame::runtime

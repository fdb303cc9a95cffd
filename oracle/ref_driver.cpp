// TEST INFRASTRUCTURE — C surface over the reference CPU backend built from /root/reference's own sources
// (oracle/Makefile, target ref). Used only by tests/ (to pin the oracle and the host harness) and by bench.py's
// cpu_baseline leg. It is compiled against the reference headers and linked with the reference objects; it is
// never part of the product.
#include <cstdint>
#include <cstring>
#include <memory>
#include <span>
#include <sstream>
#include <string>
#include <vector>

#include <frame/compiler/autograd.h>
#include <frame/compiler/pass.h>
#include <frame/compiler/pipeline.h>
#include <frame/core/dtype.h>
#include <frame/hal/allocator.h>
#include <frame/hal/backend.h>
#include <frame/hal/executable.h>
#include <frame/interop/onnx_weights.h>
#include <frame/ir/graph.h>
#include <frame/ir/memory_plan.h>
#include <frame/ir/serialization.h>
#include <frame/ops/op_registry.h>
#include <frame/runtime/compile.h>

namespace {

thread_local std::string g_error;

int set_err(const frame::Status& st) {
  g_error = std::string(st.message());
  return static_cast<int>(st.code()) == 0 ? 1 : static_cast<int>(st.code());
}

int copy_text(const std::string& s, char* out, int64_t cap, int64_t* needed) {
  if (needed != nullptr) *needed = static_cast<int64_t>(s.size()) + 1;
  if (out == nullptr || cap < static_cast<int64_t>(s.size()) + 1) return -1;
  std::memcpy(out, s.c_str(), s.size() + 1);
  return 0;
}

}  // namespace

#pragma GCC visibility push(default)
extern "C" {

const char* ref_last_error(void) { return g_error.c_str(); }

uint16_t ref_float_to_bf16(float v) { return frame::float_to_bfloat16(v).bits; }
uint16_t ref_float_to_f16(float v) { return frame::float_to_float16(v).bits; }
float ref_bf16_to_float(uint16_t b) { return frame::bfloat16_to_float(frame::bfloat16_t{b}); }
float ref_f16_to_float(uint16_t h) { return frame::float16_to_float(frame::float16_t{h}); }

// Compares the reference narrowing functions with caller-supplied ones over every 32-bit pattern.
// Returns the number of mismatches; the first mismatching input pattern goes to *first_bad.
int64_t ref_compare_narrowing_exhaustive(uint16_t (*bf16_fn)(float), uint16_t (*f16_fn)(float),
                                         uint32_t* first_bad) {
  int64_t bad = 0;
  uint32_t u = 0;
  do {
    float f;
    std::memcpy(&f, &u, 4);
    if (bf16_fn(f) != frame::float_to_bfloat16(f).bits || f16_fn(f) != frame::float_to_float16(f).bits) {
      if (bad == 0 && first_bad != nullptr) *first_bad = u;
      ++bad;
    }
    ++u;
  } while (u != 0);
  return bad;
}

// Parses `ir_text` (the reference's dump_text format), compiles it for the cpu backend and runs it on host
// buffers. Inputs are copied into reference tensors; outputs copied back into `outs` (caller sized them from
// the graph's output types).
int ref_run_graph(const char* ir_text, int n_in, const void* const* ins, int n_out, void* const* outs) {
  frame::Result<frame::ir::Graph> parsed = frame::ir::parse_text(ir_text);
  if (!parsed.is_ok()) return set_err(parsed.status());
  frame::hal::CompileOptions options;
  auto exe = frame::runtime::compile(parsed.value(), "cpu", options);
  if (!exe.is_ok()) return set_err(exe.status());
  auto backend = frame::hal::BackendRegistry::instance().get("cpu");
  if (!backend.is_ok()) return set_err(backend.status());
  frame::hal::Allocator* alloc = backend.value()->allocator(frame::cpu_device());
  const auto in_sig = exe.value()->input_signature();
  if (static_cast<int>(in_sig.size()) != n_in) {
    g_error = "ref_run_graph: input count mismatch";
    return 1;
  }
  std::vector<frame::Tensor> inputs;
  for (int i = 0; i < n_in; ++i) {
    auto t = frame::Tensor::empty(in_sig[i].shape, in_sig[i].dtype, frame::cpu_device(), *alloc);
    if (!t.is_ok()) return set_err(t.status());
    std::memcpy(t.value().raw_data(), ins[i],
                static_cast<size_t>(in_sig[i].shape.numel()) * in_sig[i].dtype.itemsize());
    inputs.push_back(t.value());
  }
  auto outputs = frame::runtime::run_with_allocated_outputs(*exe.value(), "cpu", inputs);
  if (!outputs.is_ok()) return set_err(outputs.status());
  if (static_cast<int>(outputs.value().size()) != n_out) {
    g_error = "ref_run_graph: output count mismatch";
    return 1;
  }
  for (int i = 0; i < n_out; ++i) {
    const frame::Tensor& t = outputs.value()[i];
    std::memcpy(outs[i], t.raw_data(), static_cast<size_t>(t.numel()) * t.dtype().itemsize());
  }
  return 0;
}

// Runs the reference's standard pipeline (or a single named pass when `pass_name` is non-empty) on the parsed
// graph and writes dump_text of the result.
int ref_transform_text(const char* ir_text, const char* pass_name, char* out, int64_t cap, int64_t* needed) {
  frame::Result<frame::ir::Graph> parsed = frame::ir::parse_text(ir_text);
  if (!parsed.is_ok()) return set_err(parsed.status());
  frame::compiler::PassManager manager;
  if (pass_name != nullptr && pass_name[0] != '\0') {
    manager.add(pass_name);
  } else {
    auto std_pipeline = frame::compiler::standard_pipeline("cpu");
    if (!std_pipeline.is_ok()) return set_err(std_pipeline.status());
    manager = std::move(std_pipeline.value());
  }
  const frame::Status st = manager.run(parsed.value());
  if (!st.is_ok()) return set_err(st);
  return copy_text(frame::ir::dump_text(parsed.value()), out, cap, needed);
}

// Round-trips the text through parse_text + dump_text.
// The reference's compile-time autograd on IR text (compiler::build_backward_graph / build_sgd_update_graph).
int ref_backward_text(const char* ir_text, int32_t loss_output_index, const int32_t* wrt, int32_t n_wrt, char* out,
                      int64_t cap, int64_t* needed) {
  frame::Result<frame::ir::Graph> parsed = frame::ir::parse_text(ir_text);
  if (!parsed.is_ok()) return set_err(parsed.status());
  auto t = frame::compiler::build_backward_graph(parsed.value(), loss_output_index,
                                                 std::span<const int32_t>(wrt, static_cast<size_t>(n_wrt)));
  if (!t.is_ok()) return set_err(t.status());
  return copy_text(frame::ir::dump_text(t.value()), out, cap, needed);
}

int ref_sgd_update_text(const char* ir_text, const int32_t* param_inputs, int32_t n_params, double learning_rate,
                        char* out, int64_t cap, int64_t* needed) {
  frame::Result<frame::ir::Graph> parsed = frame::ir::parse_text(ir_text);
  if (!parsed.is_ok()) return set_err(parsed.status());
  std::vector<frame::ir::TensorType> types;
  for (int32_t i = 0; i < n_params; ++i) types.push_back(parsed.value().inputs()[static_cast<size_t>(param_inputs[i])]->type());
  auto u = frame::compiler::build_sgd_update_graph(types, learning_rate);
  if (!u.is_ok()) return set_err(u.status());
  return copy_text(frame::ir::dump_text(u.value()), out, cap, needed);
}

int ref_roundtrip_text(const char* ir_text, char* out, int64_t cap, int64_t* needed) {
  frame::Result<frame::ir::Graph> parsed = frame::ir::parse_text(ir_text);
  if (!parsed.is_ok()) return set_err(parsed.status());
  return copy_text(frame::ir::dump_text(parsed.value()), out, cap, needed);
}

// Memory plan of the parsed graph as text lines "topo_index output_index offset size def last_use" plus
// "total N".
int ref_memory_plan_text(const char* ir_text, char* out, int64_t cap, int64_t* needed) {
  frame::Result<frame::ir::Graph> parsed = frame::ir::parse_text(ir_text);
  if (!parsed.is_ok()) return set_err(parsed.status());
  auto plan = frame::ir::compute_memory_plan(parsed.value());
  if (!plan.is_ok()) return set_err(plan.status());
  std::ostringstream os;
  for (const auto& [key, e] : plan.value().entries)
    os << key.first << ' ' << key.second << ' ' << e.byte_offset << ' ' << e.size_bytes << ' ' << e.def_index << ' '
       << e.last_use_index << '\n';
  os << "total " << plan.value().total_bytes << '\n';
  return copy_text(os.str(), out, cap, needed);
}

// ONNX weight exchange through the reference's own codec (src/interop/onnx_weights.cpp): save host buffers; load
// into a thread-local list read back with the ref_onnx_* accessors.
thread_local std::vector<frame::interop::NamedTensor> g_onnx;

int ref_save_onnx_weights(const char* path, int32_t n, const char* const* names, const int32_t* dtypes,
                          const int64_t* const* dims, const int32_t* ranks, const void* const* data) {
  auto b = frame::hal::BackendRegistry::instance().get(frame::kCpuBackendName);
  if (!b.is_ok()) return set_err(b.status());
  frame::hal::Allocator* alloc = b.value()->allocator(frame::cpu_device());
  std::vector<frame::interop::NamedTensor> ws;
  for (int32_t i = 0; i < n; ++i) {
    std::vector<int64_t> d(dims[i], dims[i] + ranks[i]);
    auto t = frame::Tensor::empty(frame::Shape(d), frame::DType(static_cast<frame::DTypeCode>(dtypes[i])),
                                  frame::cpu_device(), *alloc);
    if (!t.is_ok()) return set_err(t.status());
    std::memcpy(t.value().raw_data(), data[i], static_cast<size_t>(t.value().numel()) * t.value().dtype().itemsize());
    ws.push_back(frame::interop::NamedTensor{names[i], t.value()});
  }
  frame::Status st = frame::interop::save_onnx_weights(path, ws);
  return st.is_ok() ? 0 : set_err(st);
}

int ref_load_onnx_weights(const char* path) {
  auto b = frame::hal::BackendRegistry::instance().get(frame::kCpuBackendName);
  if (!b.is_ok()) return set_err(b.status());
  auto r = frame::interop::load_onnx_weights(path, *b.value()->allocator(frame::cpu_device()));
  if (!r.is_ok()) return set_err(r.status());
  g_onnx = std::move(r.value());
  return 0;
}
int32_t ref_onnx_count(void) { return static_cast<int32_t>(g_onnx.size()); }
const char* ref_onnx_name(int32_t i) { return g_onnx[static_cast<size_t>(i)].name.c_str(); }
int32_t ref_onnx_dtype(int32_t i) { return static_cast<int32_t>(g_onnx[static_cast<size_t>(i)].tensor.dtype().code()); }
int32_t ref_onnx_rank(int32_t i) { return static_cast<int32_t>(g_onnx[static_cast<size_t>(i)].tensor.shape().rank()); }
int64_t ref_onnx_dim(int32_t i, int32_t k) { return g_onnx[static_cast<size_t>(i)].tensor.shape().dim(k); }
const void* ref_onnx_data(int32_t i) { return g_onnx[static_cast<size_t>(i)].tensor.raw_data(); }

}  // extern "C"
#pragma GCC visibility pop

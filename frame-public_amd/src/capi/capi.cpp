// C entry points of libframe.so (include/frame_capi.h) over the C++20 host API.
#pragma GCC visibility push(default)
#include "frame_capi.h"
#pragma GCC visibility pop

#include <cstdlib>
#include <cstring>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include <frame/compiler/autograd.h>
#include <frame/compiler/pipeline.h>
#include <frame/core/tensor.h>
#include <frame/hal/allocator.h>
#include <frame/hal/backend.h>
#include <frame/hal/event.h>
#include <frame/hal/executable.h>
#include <frame/hal/stream.h>
#include <frame/ir/graph.h>
#include <frame/ir/memory_plan.h>
#include <frame/interop/onnx_weights.h>
#include <frame/ir/serialization.h>
#include <frame/runtime/compile.h>

#include "backends/hip/hip_backend.h"

struct frame_tensor {
  frame::Tensor t;
  frame::hal::Backend* backend;
};
struct frame_stream {
  std::unique_ptr<frame::hal::Stream> s;
};
struct frame_event {
  std::unique_ptr<frame::hal::Event> e;
};
struct frame_onnx_weights {
  std::vector<frame::interop::NamedTensor> items;
};
struct frame_executable {
  std::shared_ptr<frame::hal::Executable> exe;
  std::string backend;
};

namespace {

// Host memory for cpu tensors (ONNX weights): 64-byte aligned blocks from the C library. The hip plugin's library
// registers no cpu backend, so the C API brings its own host allocator.
class HostAllocator final : public frame::hal::Allocator {
 public:
  frame::Result<void*> allocate(size_t bytes, size_t alignment) override {
    if (bytes == 0) return frame::Status::make(frame::ErrorCode::kInvalidArgument, "host allocate: 0 bytes");
    if (alignment == 0 || (alignment & (alignment - 1)) != 0 || alignment > 64)
      return frame::Status::make(frame::ErrorCode::kInvalidArgument, "host allocate: bad alignment");
    void* p = std::aligned_alloc(64, (bytes + 63) / 64 * 64);
    if (p == nullptr) return frame::Status::make(frame::ErrorCode::kOutOfMemory, "host allocate failed");
    return p;
  }
  void deallocate(void* p) override { std::free(p); }
};

HostAllocator& host_allocator() {
  static HostAllocator a;  // process lifetime: tensors it backs may be released at any time
  return a;
}

thread_local std::string g_error;

int fail(const frame::Status& s) {
  g_error = std::string(s.message());
  const int code = static_cast<int>(s.code());
  return code == 0 ? static_cast<int>(frame::ErrorCode::kInternal) : code;
}

int fail_msg(const std::string& m) {
  g_error = m;
  return static_cast<int>(frame::ErrorCode::kInvalidArgument);
}

int text_out(const std::string& s, char* out, int64_t cap, int64_t* needed) {
  if (needed != nullptr) *needed = static_cast<int64_t>(s.size()) + 1;
  if (out == nullptr || cap < static_cast<int64_t>(s.size()) + 1) return -1;
  std::memcpy(out, s.c_str(), s.size() + 1);
  return 0;
}

frame::Result<frame::hal::Backend*> backend_of(const char* name) {
  if (name == nullptr) return frame::Status::make(frame::ErrorCode::kInvalidArgument, "backend name is null");
  return frame::hal::BackendRegistry::instance().get(name);
}

std::vector<frame::Tensor> unwrap(frame_tensor* const* ts, int32_t n) {
  std::vector<frame::Tensor> v;
  for (int32_t i = 0; i < n; ++i) v.push_back(ts[i]->t);
  return v;
}

}  // namespace

#pragma GCC visibility push(default)
extern "C" {

const char* frame_last_error(void) { return g_error.c_str(); }

int frame_backends(char* out, int64_t cap, int64_t* needed) {
  std::string s;
  for (std::string_view n : frame::hal::BackendRegistry::instance().available()) s += (s.empty() ? "" : ",") + std::string(n);
  return text_out(s, out, cap, needed);
}

int frame_device_count(const char* backend, int32_t* count) {
  auto b = backend_of(backend);
  if (!b.is_ok()) return fail(b.status());
  auto n = b.value()->device_count();
  if (!n.is_ok()) return fail(n.status());
  *count = n.value();
  return 0;
}

int frame_tensor_empty(const char* backend, int32_t device, int32_t dtype, const int64_t* dims, int32_t rank,
                       frame_tensor** out) {
  if (out == nullptr || rank < 0 || (rank > 0 && dims == nullptr)) return fail_msg("frame_tensor_empty: bad arguments");
  if (dtype < 0 || dtype >= static_cast<int32_t>(frame::DTypeCode::kCount)) return fail_msg("frame_tensor_empty: bad dtype");
  auto b = backend_of(backend);
  if (!b.is_ok()) return fail(b.status());
  const frame::Device dev{b.value()->name(), device};
  frame::hal::Allocator* a = b.value()->allocator(dev);
  if (a == nullptr) return fail_msg("frame_tensor_empty: backend has no allocator for device " + std::to_string(device));
  auto t = frame::Tensor::empty(frame::Shape(std::vector<int64_t>(dims, dims + rank)),
                                frame::DType(static_cast<frame::DTypeCode>(dtype)), dev, *a);
  if (!t.is_ok()) return fail(t.status());
  *out = new frame_tensor{t.value(), b.value()};
  return 0;
}

int frame_tensor_empty_at(const char* backend, int32_t device, int32_t dtype, const int64_t* dims, int32_t rank,
                          int64_t byte_offset, frame_tensor** out) {
  if (out == nullptr || rank < 0 || (rank > 0 && dims == nullptr) || byte_offset < 0)
    return fail_msg("frame_tensor_empty_at: bad arguments");
  if (dtype < 0 || dtype >= static_cast<int32_t>(frame::DTypeCode::kCount)) return fail_msg("frame_tensor_empty_at: bad dtype");
  const frame::DType dt(static_cast<frame::DTypeCode>(dtype));
  if (byte_offset % static_cast<int64_t>(dt.itemsize()) != 0)
    return fail_msg("frame_tensor_empty_at: byte_offset is not a multiple of the element size");
  auto b = backend_of(backend);
  if (!b.is_ok()) return fail(b.status());
  const frame::Device dev{b.value()->name(), device};
  frame::hal::Allocator* a = b.value()->allocator(dev);
  if (a == nullptr) return fail_msg("frame_tensor_empty_at: backend has no allocator for device " + std::to_string(device));
  const frame::Shape shape(std::vector<int64_t>(dims, dims + rank));
  const size_t bytes = static_cast<size_t>(shape.numel()) * dt.itemsize() + static_cast<size_t>(byte_offset);
  auto st = frame::Storage::allocate(*a, bytes == 0 ? 1 : bytes, frame::kDefaultAlignment, dev);
  if (!st.is_ok()) return fail(st.status());
  *out = new frame_tensor{frame::Tensor::from_storage_slice(st.value(), static_cast<size_t>(byte_offset), shape, dt, dev),
                          b.value()};
  return 0;
}

void frame_tensor_free(frame_tensor* t) { delete t; }
void* frame_tensor_data(frame_tensor* t) { return t == nullptr ? nullptr : t->t.raw_data(); }
int64_t frame_tensor_nbytes(const frame_tensor* t) {
  return t == nullptr ? 0 : t->t.numel() * static_cast<int64_t>(t->t.dtype().itemsize());
}

int frame_tensor_upload(frame_tensor* t, const void* host, size_t bytes) {
  if (t == nullptr || static_cast<int64_t>(bytes) != frame_tensor_nbytes(t)) return fail_msg("frame_tensor_upload: size mismatch");
  frame::Status s = t->backend->copy(t->t.raw_data(), t->t.device(), host, frame::cpu_device(), bytes, nullptr);
  return s.is_ok() ? 0 : fail(s);
}

int frame_tensor_download(const frame_tensor* t, void* host, size_t bytes) {
  if (t == nullptr || static_cast<int64_t>(bytes) != frame_tensor_nbytes(t)) return fail_msg("frame_tensor_download: size mismatch");
  frame::Status s = t->backend->copy(host, frame::cpu_device(), t->t.raw_data(), t->t.device(), bytes, nullptr);
  return s.is_ok() ? 0 : fail(s);
}

int frame_stream_create(const char* backend, int32_t device, frame_stream** out) {
  auto b = backend_of(backend);
  if (!b.is_ok()) return fail(b.status());
  auto s = b.value()->create_stream(frame::Device{b.value()->name(), device});
  if (!s.is_ok()) return fail(s.status());
  *out = new frame_stream{std::move(s.value())};
  return 0;
}
void frame_stream_destroy(frame_stream* s) { delete s; }
int frame_stream_synchronize(frame_stream* s) {
  frame::Status st = s->s->synchronize();
  return st.is_ok() ? 0 : fail(st);
}
void* frame_stream_native(frame_stream* s) { return s->s->native_handle(); }

int frame_event_create(const char* backend, int32_t device, frame_event** out) {
  auto b = backend_of(backend);
  if (!b.is_ok()) return fail(b.status());
  auto e = b.value()->create_event(frame::Device{b.value()->name(), device});
  if (!e.is_ok()) return fail(e.status());
  *out = new frame_event{std::move(e.value())};
  return 0;
}
void frame_event_destroy(frame_event* e) { delete e; }
int frame_event_record(frame_event* e, frame_stream* s) {
  frame::Status st = s->s->record(*e->e);
  return st.is_ok() ? 0 : fail(st);
}
int frame_event_synchronize(frame_event* e) {
  frame::Status st = e->e->synchronize();
  return st.is_ok() ? 0 : fail(st);
}

int frame_compile(const char* ir_text, const char* backend, int32_t opt_level, frame_executable** out) {
  if (ir_text == nullptr || backend == nullptr || out == nullptr) return fail_msg("frame_compile: null argument");
  auto g = frame::ir::parse_text(ir_text);
  if (!g.is_ok()) return fail(g.status());
  frame::hal::CompileOptions opts;
  opts.opt_level = opt_level;
  auto e = frame::runtime::compile(g.value(), backend, opts);
  if (!e.is_ok()) return fail(e.status());
  *out = new frame_executable{e.value(), backend};
  return 0;
}

int frame_backend_compile(const char* ir_text, const char* backend, int32_t opt_level, frame_executable** out) {
  if (ir_text == nullptr || backend == nullptr || out == nullptr) return fail_msg("frame_backend_compile: null argument");
  auto g = frame::ir::parse_text(ir_text);
  if (!g.is_ok()) return fail(g.status());
  auto b = backend_of(backend);
  if (!b.is_ok()) return fail(b.status());
  frame::hal::CompileOptions opts;
  opts.opt_level = opt_level;
  auto e = b.value()->compile(g.value(), opts);
  if (!e.is_ok()) return fail(e.status());
  *out = new frame_executable{std::shared_ptr<frame::hal::Executable>(std::move(e.value())), backend};
  return 0;
}

void frame_executable_free(frame_executable* e) { delete e; }
int32_t frame_executable_num_inputs(const frame_executable* e) {
  return static_cast<int32_t>(e->exe->input_signature().size());
}
int32_t frame_executable_num_outputs(const frame_executable* e) {
  return static_cast<int32_t>(e->exe->output_signature().size());
}

int frame_executable_io_spec(const frame_executable* e, int32_t is_output, int32_t index, int32_t* dtype, int64_t* dims,
                             int32_t* rank) {
  const auto sig = is_output ? e->exe->output_signature() : e->exe->input_signature();
  if (index < 0 || index >= static_cast<int32_t>(sig.size())) return fail_msg("frame_executable_io_spec: index out of range");
  const auto& s = sig[static_cast<size_t>(index)];
  if (s.shape.rank() > 8) return fail_msg("frame_executable_io_spec: rank above 8");
  *dtype = static_cast<int32_t>(s.dtype.code());
  *rank = static_cast<int32_t>(s.shape.rank());
  for (int64_t i = 0; i < s.shape.rank(); ++i) dims[i] = s.shape.dim(i);
  return 0;
}

int frame_executable_run(frame_executable* e, frame_tensor* const* inputs, int32_t n_in, frame_tensor* const* outputs,
                         int32_t n_out, frame_stream* stream) {
  if (e == nullptr || stream == nullptr) return fail_msg("frame_executable_run: null argument");
  std::vector<frame::Tensor> ins = unwrap(inputs, n_in), outs = unwrap(outputs, n_out);
  frame::Status s = e->exe->run(ins, outs, *stream->s);
  return s.is_ok() ? 0 : fail(s);
}

int frame_executable_run_repeat(frame_executable* e, frame_tensor* const* input_sets, int32_t n_sets, int32_t n_in,
                                frame_tensor* const* outputs, int32_t n_out, frame_stream* stream, int32_t iterations) {
  if (e == nullptr || stream == nullptr || n_sets < 1 || n_in < 0 || n_out < 0 || iterations < 0 ||
      (n_in > 0 && input_sets == nullptr) || (n_out > 0 && outputs == nullptr))
    return fail_msg("frame_executable_run_repeat: bad argument");
  std::vector<std::vector<frame::Tensor>> sets;
  for (int32_t k = 0; k < n_sets; ++k) sets.push_back(unwrap(input_sets + static_cast<size_t>(k) * n_in, n_in));
  std::vector<frame::Tensor> outs = unwrap(outputs, n_out);
  for (int32_t i = 0; i < iterations; ++i) {
    frame::Status s = e->exe->run(sets[static_cast<size_t>(i % n_sets)], outs, *stream->s);
    if (!s.is_ok()) return fail(s);
  }
  return 0;
}

int frame_run_with_allocated_outputs(frame_executable* e, frame_tensor* const* inputs, int32_t n_in,
                                     frame_tensor** outputs, int32_t n_out) {
  std::vector<frame::Tensor> ins = unwrap(inputs, n_in);
  auto r = frame::runtime::run_with_allocated_outputs(*e->exe, e->backend, ins);
  if (!r.is_ok()) return fail(r.status());
  if (static_cast<int32_t>(r.value().size()) != n_out) return fail_msg("frame_run_with_allocated_outputs: output count mismatch");
  auto b = backend_of(e->backend.c_str());
  for (int32_t i = 0; i < n_out; ++i) outputs[i] = new frame_tensor{r.value()[static_cast<size_t>(i)], b.value()};
  return 0;
}

int frame_hip_run_tapped(frame_executable* e, frame_tensor* const* inputs, int32_t n_in, frame_tensor* const* outputs,
                         int32_t n_out, frame_stream* stream, int32_t n_taps, const int32_t* steps,
                         const int32_t* output_index, void* const* host, const int64_t* bytes) {
  if (e == nullptr || stream == nullptr || n_taps < 0 ||
      (n_taps > 0 && (steps == nullptr || output_index == nullptr || host == nullptr || bytes == nullptr)))
    return fail_msg("frame_hip_run_tapped: null argument");
  if (e->backend != frame::kHipBackendName) return fail_msg("frame_hip_run_tapped: not a hip executable");
  std::vector<frame::backends::hip::HipStepTap> taps;
  for (int32_t i = 0; i < n_taps; ++i) {
    if (steps[i] < 0 || output_index[i] < 0 || bytes[i] < 0 || (bytes[i] > 0 && host[i] == nullptr))
      return fail_msg("frame_hip_run_tapped: bad tap " + std::to_string(i));
    taps.push_back({static_cast<size_t>(steps[i]), static_cast<size_t>(output_index[i]), host[i],
                    static_cast<size_t>(bytes[i])});
  }
  std::vector<frame::Tensor> ins = unwrap(inputs, n_in), outs = unwrap(outputs, n_out);
  frame::Status s = frame::backends::hip::hip_run_tapped(*e->exe, ins, outs, *stream->s, taps);
  return s.is_ok() ? 0 : fail(s);
}

int frame_hip_executable_steps(const frame_executable* e, char* out, int64_t cap, int64_t* needed) {
  if (e == nullptr) return fail_msg("frame_hip_executable_steps: null argument");
  if (e->backend != frame::kHipBackendName) return fail_msg("frame_hip_executable_steps: not a hip executable");
  return text_out(frame::backends::hip::hip_executable_steps(*e->exe), out, cap, needed);
}

int64_t frame_compile_cache_size(void) { return static_cast<int64_t>(frame::runtime::compilation_cache_size()); }

int frame_transform_text(const char* ir_text, const char* pass_name, char* out, int64_t cap, int64_t* needed) {
  auto g = frame::ir::parse_text(ir_text);
  if (!g.is_ok()) return fail(g.status());
  frame::compiler::PassManager pm;
  if (pass_name != nullptr && pass_name[0] != '\0') {
    pm.add(pass_name);
  } else {
    auto p = frame::compiler::standard_pipeline("");
    if (!p.is_ok()) return fail(p.status());
    pm = std::move(p.value());
  }
  frame::Status s = pm.run(g.value());
  if (!s.is_ok()) return fail(s);
  return text_out(frame::ir::dump_text(g.value()), out, cap, needed);
}

int frame_hip_lowered_text(const char* ir_text, int32_t opt_level, char* out, int64_t cap, int64_t* needed) {
  auto g = frame::ir::parse_text(ir_text);
  if (!g.is_ok()) return fail(g.status());
  auto p = frame::compiler::standard_pipeline(frame::kHipBackendName);
  if (!p.is_ok()) return fail(p.status());
  frame::Status s = p.value().run(g.value());
  if (!s.is_ok()) return fail(s);
  auto lowered = frame::backends::hip::lower_for_hip(g.value(), opt_level);
  if (!lowered.is_ok()) return fail(lowered.status());
  return text_out(frame::ir::dump_text(lowered.value()), out, cap, needed);
}

int frame_backward_text(const char* ir_text, int32_t loss_output_index, const int32_t* wrt, int32_t n_wrt, char* out,
                        int64_t cap, int64_t* needed) {
  auto g = frame::ir::parse_text(ir_text);
  if (!g.is_ok()) return fail(g.status());
  std::span<const int32_t> idx(wrt, static_cast<size_t>(n_wrt < 0 ? 0 : n_wrt));
  auto t = frame::compiler::build_backward_graph(g.value(), loss_output_index, idx);
  if (!t.is_ok()) return fail(t.status());
  return text_out(frame::ir::dump_text(t.value()), out, cap, needed);
}

int frame_sgd_update_text(const char* ir_text, const int32_t* param_inputs, int32_t n_params, double learning_rate,
                          char* out, int64_t cap, int64_t* needed) {
  auto g = frame::ir::parse_text(ir_text);
  if (!g.is_ok()) return fail(g.status());
  std::vector<frame::ir::TensorType> types;
  for (int32_t i = 0; i < n_params; ++i) {
    const int32_t k = param_inputs[i];
    if (k < 0 || static_cast<size_t>(k) >= g.value().inputs().size())
      return fail(frame::Status::make(frame::ErrorCode::kInvalidArgument,
                                      "frame_sgd_update_text: param input index " + std::to_string(k) + " is out of range"));
    types.push_back(g.value().inputs()[static_cast<size_t>(k)]->type());
  }
  auto u = frame::compiler::build_sgd_update_graph(types, learning_rate);
  if (!u.is_ok()) return fail(u.status());
  return text_out(frame::ir::dump_text(u.value()), out, cap, needed);
}

int frame_roundtrip_text(const char* ir_text, char* out, int64_t cap, int64_t* needed) {
  auto g = frame::ir::parse_text(ir_text);
  if (!g.is_ok()) return fail(g.status());
  return text_out(frame::ir::dump_text(g.value()), out, cap, needed);
}

int frame_memory_plan_text(const char* ir_text, char* out, int64_t cap, int64_t* needed) {
  auto g = frame::ir::parse_text(ir_text);
  if (!g.is_ok()) return fail(g.status());
  auto plan = frame::ir::compute_memory_plan(g.value());
  if (!plan.is_ok()) return fail(plan.status());
  std::ostringstream os;
  for (const auto& [k, e] : plan.value().entries)
    os << k.first << ' ' << k.second << ' ' << e.byte_offset << ' ' << e.size_bytes << ' ' << e.def_index << ' '
       << e.last_use_index << '\n';
  os << "total " << plan.value().total_bytes << '\n';
  return text_out(os.str(), out, cap, needed);
}

int frame_launch(const char* node_ir_text, const char* backend, frame_tensor* const* inputs, int32_t n_in,
                 frame_tensor* const* outputs, int32_t n_out, frame_stream* stream) {
  auto g = frame::ir::parse_text(node_ir_text);
  if (!g.is_ok()) return fail(g.status());
  const frame::ir::Node* node = nullptr;
  for (const frame::ir::Node* n : g.value().topological_order()) {
    if (n->op() == frame::ir::kGraphInputOp) continue;
    if (node != nullptr) return fail_msg("frame_launch: the text holds more than one operator node");
    node = n;
  }
  if (node == nullptr) return fail_msg("frame_launch: the text holds no operator node");
  auto b = backend_of(backend);
  if (!b.is_ok()) return fail(b.status());
  std::vector<frame::Tensor> ins = unwrap(inputs, n_in), outs = unwrap(outputs, n_out);
  frame::hal::KernelInvocation inv{node->op(), ins, outs, &node->attrs(), frame::Device{b.value()->name(), 0}};
  frame::Status s = b.value()->launch(inv, stream ? stream->s.get() : nullptr);
  return s.is_ok() ? 0 : fail(s);
}

int frame_save_onnx_weights(const char* path, int32_t n, const char* const* names, const int32_t* dtypes,
                            const int64_t* const* dims, const int32_t* ranks, const void* const* data) {
  if (path == nullptr || n < 0 || (n > 0 && (names == nullptr || dtypes == nullptr || dims == nullptr ||
                                             ranks == nullptr || data == nullptr)))
    return fail_msg("frame_save_onnx_weights: null argument");
  std::vector<frame::interop::NamedTensor> ws;
  for (int32_t i = 0; i < n; ++i) {
    if (ranks[i] < 0 || (ranks[i] > 0 && dims[i] == nullptr)) return fail_msg("frame_save_onnx_weights: bad shape");
    if (names[i] == nullptr) return fail_msg("frame_save_onnx_weights: null name");
    if (dtypes[i] != static_cast<int32_t>(frame::DTypeCode::kFloat32) &&
        dtypes[i] != static_cast<int32_t>(frame::DTypeCode::kFloat16) &&
        dtypes[i] != static_cast<int32_t>(frame::DTypeCode::kBFloat16))
      return fail_msg("frame_save_onnx_weights: dtype code " + std::to_string(dtypes[i]) +
                      " is not float32 (0), float16 (2) or bfloat16 (3)");
    std::vector<int64_t> d(dims[i], dims[i] + ranks[i]);
    auto t = frame::Tensor::empty(frame::Shape(d), frame::DType(static_cast<frame::DTypeCode>(dtypes[i])),
                                  frame::cpu_device(), host_allocator());
    if (!t.is_ok()) return fail(t.status());
    const size_t nbytes = static_cast<size_t>(t.value().numel()) * t.value().dtype().itemsize();
    if (nbytes > 0 && data[i] == nullptr) return fail_msg("frame_save_onnx_weights: null data for a non-empty tensor");
    if (nbytes > 0) std::memcpy(t.value().raw_data(), data[i], nbytes);
    ws.push_back(frame::interop::NamedTensor{names[i], t.value()});
  }
  frame::Status st = frame::interop::save_onnx_weights(path, ws);
  return st.is_ok() ? 0 : fail(st);
}

int frame_load_onnx_weights(const char* path, frame_onnx_weights** out) {
  if (path == nullptr || out == nullptr) return fail_msg("frame_load_onnx_weights: null argument");
  auto r = frame::interop::load_onnx_weights(path, host_allocator());
  if (!r.is_ok()) return fail(r.status());
  *out = new frame_onnx_weights{std::move(r.value())};
  return 0;
}
int32_t frame_onnx_count(const frame_onnx_weights* w) { return static_cast<int32_t>(w->items.size()); }
const char* frame_onnx_name(const frame_onnx_weights* w, int32_t i) { return w->items[static_cast<size_t>(i)].name.c_str(); }
int32_t frame_onnx_dtype(const frame_onnx_weights* w, int32_t i) {
  return static_cast<int32_t>(w->items[static_cast<size_t>(i)].tensor.dtype().code());
}
int32_t frame_onnx_rank(const frame_onnx_weights* w, int32_t i) {
  return static_cast<int32_t>(w->items[static_cast<size_t>(i)].tensor.shape().rank());
}
int64_t frame_onnx_dim(const frame_onnx_weights* w, int32_t i, int32_t k) {
  return w->items[static_cast<size_t>(i)].tensor.shape().dim(k);
}
const void* frame_onnx_data(const frame_onnx_weights* w, int32_t i) { return w->items[static_cast<size_t>(i)].tensor.raw_data(); }
void frame_onnx_free(frame_onnx_weights* w) { delete w; }

int frame_backend_copy(const char* backend, void* dst, const char* dst_backend, int32_t dst_index, const void* src,
                       const char* src_backend, int32_t src_index, size_t bytes, frame_stream* stream) {
  auto b = backend_of(backend);
  if (!b.is_ok()) return fail(b.status());
  auto dev = [](const char* name, int32_t index) -> frame::Result<frame::Device> {
    if (name == nullptr) return frame::Status::make(frame::ErrorCode::kInvalidArgument, "device backend is null");
    const std::string_view n(name);
    if (n == frame::kCpuBackendName) return frame::Device{frame::kCpuBackendName, index};
    if (n == frame::kHipBackendName) return frame::Device{frame::kHipBackendName, index};
    return frame::Status::make(frame::ErrorCode::kInvalidArgument, "unknown device backend '" + std::string(n) + "'");
  };
  auto d = dev(dst_backend, dst_index);
  if (!d.is_ok()) return fail(d.status());
  auto s = dev(src_backend, src_index);
  if (!s.is_ok()) return fail(s.status());
  frame::Status st = b.value()->copy(dst, d.value(), src, s.value(), bytes, stream ? stream->s.get() : nullptr);
  return st.is_ok() ? 0 : fail(st);
}

int frame_hip_allocator_stats(int32_t device, uint64_t out[6]) {
  auto b = backend_of(frame::kHipBackendName.data());
  if (!b.is_ok()) return fail(b.status());
  auto* a = dynamic_cast<frame::backends::hip::HipAllocator*>(b.value()->allocator(frame::Device{frame::kHipBackendName, device}));
  if (a == nullptr) return fail_msg("frame_hip_allocator_stats: no hip allocator for device " + std::to_string(device));
  const auto st = a->stats();
  out[0] = st.live_bytes;
  out[1] = st.cached_bytes;
  out[2] = st.pending_bytes;
  out[3] = st.device_allocations;
  out[4] = st.device_syncs;
  out[5] = st.fence_waits;
  return 0;
}

}  // extern "C"
#pragma GCC visibility pop

// pybind11 module `frame_hip_py`: the Python surface of the reference (python/src/bind_runtime.cpp:33-56 and
// bind_interop.cpp:38-74) over this repository's host library, so that a Python caller compiles and runs a graph on
// the `hip` backend the way the reference's `frame.compile(graph, backend).run(inputs)` does:
//   compile(graph_text, backend) -> Executable         runtime::compile (GIL released)
//   Executable.run(list[Tensor]) -> list[Tensor]        runtime::run_with_allocated_outputs (GIL released)
//   Tensor.from_numpy(backend, dtype, array), Tensor.numpy(), .shape, .dtype, .backend
//   save_onnx_weights(path, dict[str, Tensor]), load_onnx_weights(path) -> dict[str, Tensor]   (cpu tensors)
// The graph is given as IR text (ir::parse_text), the form every other entry point of this repository takes.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include <frame/core/device.h>
#include <frame/core/dtype.h>
#include <frame/core/tensor.h>
#include <frame/hal/allocator.h>
#include <frame/hal/backend.h>
#include <frame/hal/executable.h>
#include <frame/interop/onnx_weights.h>
#include <frame/ir/serialization.h>
#include <frame/runtime/compile.h>

namespace py = pybind11;

namespace {

// Status -> Python exception, with the status message as the exception's text unchanged. The exception types are
// the reference binding's (python/src/translate_status.cpp:29-47): invalid argument -> ValueError, not found ->
// KeyError, unimplemented -> NotImplementedError, out of memory -> MemoryError, every other code -> RuntimeError.
PyObject* exception_type(frame::ErrorCode code) {
  switch (code) {
    case frame::ErrorCode::kInvalidArgument: return PyExc_ValueError;
    case frame::ErrorCode::kNotFound: return PyExc_KeyError;
    case frame::ErrorCode::kUnimplemented: return PyExc_NotImplementedError;
    case frame::ErrorCode::kOutOfMemory: return PyExc_MemoryError;
    default: return PyExc_RuntimeError;
  }
}
// Thrown where a Status fails (possibly with the GIL released, inside compile and run) and turned into the Python
// exception by the translator registered in the module, which runs with the GIL held.
struct StatusError {
  frame::ErrorCode code;
  std::string message;
};
[[noreturn]] void raise(const frame::Status& st) { throw StatusError{st.code(), std::string(st.message())}; }
template <typename T>
T unwrap(frame::Result<T> r) {
  if (!r.is_ok()) raise(r.status());
  return std::move(r.value());
}
void check(const frame::Status& st) {
  if (!st.is_ok()) raise(st);
}

class HostAllocator final : public frame::hal::Allocator {
 public:
  frame::Result<void*> allocate(size_t bytes, size_t alignment) override {
    if (bytes == 0 || alignment == 0 || alignment > 64 || (alignment & (alignment - 1)) != 0)
      return frame::Status::make(frame::ErrorCode::kInvalidArgument, "host allocator: bad request");
    void* p = std::aligned_alloc(64, (bytes + 63) / 64 * 64);
    if (p == nullptr) return frame::Status::make(frame::ErrorCode::kOutOfMemory, "host allocator: out of memory");
    return p;
  }
  void deallocate(void* p) override { std::free(p); }
};
HostAllocator& host_allocator() {
  static HostAllocator a;
  return a;
}

frame::Device device_of(const std::string& backend) {
  if (backend == frame::kCpuBackendName) return frame::cpu_device();
  if (backend == frame::kHipBackendName) return frame::Device{frame::kHipBackendName, 0};
  throw py::value_error("unknown backend '" + backend + "'");
}

frame::hal::Backend* hip_backend() { return unwrap(frame::hal::BackendRegistry::instance().get(frame::kHipBackendName)); }

py::dtype np_dtype(frame::DType d) {
  switch (d.code()) {
    case frame::DTypeCode::kFloat32: return py::dtype::of<float>();
    case frame::DTypeCode::kFloat16:
    case frame::DTypeCode::kBFloat16: return py::dtype::of<uint16_t>();  // storage bits
    default: throw py::value_error("dtype '" + std::string(d.name()) + "' has no numpy storage type here");
  }
}

frame::Tensor tensor_from_numpy(const std::string& backend, int dtype, py::array array) {
  const frame::DType d(static_cast<frame::DTypeCode>(dtype));
  py::array a = py::array::ensure(array, py::array::c_style);
  if (!a || a.dtype().itemsize() != static_cast<py::ssize_t>(d.itemsize()))
    throw py::value_error("array item size does not match the dtype");
  std::vector<int64_t> dims(a.shape(), a.shape() + a.ndim());
  const frame::Device dev = device_of(backend);
  frame::hal::Allocator* alloc = backend == frame::kCpuBackendName ? &host_allocator() : hip_backend()->allocator(dev);
  frame::Tensor t = unwrap(frame::Tensor::empty(frame::Shape(dims), d, dev, *alloc));
  const size_t n = static_cast<size_t>(t.numel()) * d.itemsize();
  if (n == 0) return t;
  if (backend == frame::kCpuBackendName)
    std::memcpy(t.raw_data(), a.data(), n);
  else
    check(hip_backend()->copy(t.raw_data(), dev, a.data(), frame::cpu_device(), n, nullptr));
  return t;
}

py::array tensor_to_numpy(const frame::Tensor& t) {
  std::vector<py::ssize_t> shape(t.shape().dims().begin(), t.shape().dims().end());
  py::array out(np_dtype(t.dtype()), shape);
  const size_t n = static_cast<size_t>(t.numel()) * t.dtype().itemsize();
  if (n == 0) return out;
  if (t.device().backend == frame::kCpuBackendName)
    std::memcpy(out.mutable_data(), t.raw_data(), n);
  else
    check(hip_backend()->copy(out.mutable_data(), frame::cpu_device(), t.raw_data(), t.device(), n, nullptr));
  return out;
}

struct BoundExecutable {
  std::shared_ptr<frame::hal::Executable> executable;
  std::string backend;
};

}  // namespace

PYBIND11_MODULE(frame_hip_py, m) {
  m.doc() = "Frame's compiled-graph path from Python: compile(graph_text, backend).run(inputs)";
  py::register_exception_translator([](std::exception_ptr p) {
    try {
      if (p) std::rethrow_exception(p);
    } catch (const StatusError& e) {
      PyErr_SetString(exception_type(e.code), e.message.c_str());
    }
  });
  py::class_<frame::Tensor>(m, "Tensor")
      .def_static("from_numpy", &tensor_from_numpy, py::arg("backend"), py::arg("dtype"), py::arg("array"))
      .def("numpy", &tensor_to_numpy)
      .def_property_readonly("shape", [](const frame::Tensor& t) { return t.shape().dims(); })
      .def_property_readonly("dtype", [](const frame::Tensor& t) { return static_cast<int>(t.dtype().code()); })
      .def_property_readonly("backend", [](const frame::Tensor& t) { return std::string(t.device().backend); });
  py::class_<BoundExecutable>(m, "Executable")
      .def("run",
           [](BoundExecutable& self, const std::vector<frame::Tensor>& inputs) {
             return unwrap(frame::runtime::run_with_allocated_outputs(*self.executable, self.backend, inputs));
           },
           py::arg("inputs"), py::call_guard<py::gil_scoped_release>());
  m.def("compile",
        [](const std::string& graph_text, const std::string& backend) {
          frame::ir::Graph g = unwrap(frame::ir::parse_text(graph_text));
          return BoundExecutable{unwrap(frame::runtime::compile(g, backend, frame::hal::CompileOptions{})), backend};
        },
        py::arg("graph"), py::arg("backend"), py::call_guard<py::gil_scoped_release>());
  m.def("save_onnx_weights",
        [](const std::string& path, const py::dict& weights) {
          std::vector<frame::interop::NamedTensor> ws;
          for (const auto& kv : weights) ws.push_back({kv.first.cast<std::string>(), kv.second.cast<frame::Tensor>()});
          check(frame::interop::save_onnx_weights(path, ws));
        },
        py::arg("path"), py::arg("weights"));
  m.def("load_onnx_weights",
        [](const std::string& path) {
          py::dict out;
          for (auto& w : unwrap(frame::interop::load_onnx_weights(path, host_allocator())))
            out[py::str(w.name)] = py::cast(std::move(w.tensor));
          return out;
        },
        py::arg("path"));
  // Test hook: raises what a Status of `code` (a frame::ErrorCode ordinal) with `message` turns into; 0 returns.
  m.def("_raise_status",
        [](int code, const std::string& message) {
          if (code < 0 || code > static_cast<int>(frame::ErrorCode::kDeviceError)) throw py::value_error("bad error code");
          const frame::Status st = frame::Status::make(static_cast<frame::ErrorCode>(code), message);
          if (!st.is_ok()) raise(st);
        },
        py::arg("code"), py::arg("message"));
}

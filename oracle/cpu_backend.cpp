// TEST INFRASTRUCTURE — the CPU parity oracle registered as Frame's `cpu` backend inside libframe.so.
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it (lib/liboracle_cpu.so); the
// product never links or calls it.
//
// Mirrors the reference's CPU backend (src/backends/cpu/cpu_backend.cpp:21-146: one device, synchronous no-op
// stream and events, aligned host allocator, memmove copy; src/backends/cpu/cpu_executable.cpp:42-131: a fresh
// arena per run, graph outputs allocated per run and copied out). Its kernels are the single-threaded
// restatement in cpu_kernels.cpp, so a graph compiled for `cpu` here computes what the reference's cpu backend
// computes; tests pin that against oracle/_ref (the reference built from its own sources).
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include <frame/core/tensor.h>
#include <frame/hal/allocator.h>
#include <frame/hal/backend.h>
#include <frame/hal/event.h>
#include <frame/hal/executable.h>
#include <frame/hal/stream.h>
#include <frame/ir/graph.h>
#include <frame/ops/constant_utils.h>
#include <frame/ops/executable_plan.h>
#include <frame/ops/fused_elementwise_utils.h>
#include <frame/ops/kernel_registry.h>

#include "cpu_kernels.h"

namespace oracle_cpu {

using namespace frame;

class CpuStream final : public hal::Stream {
 public:
  Status synchronize() override { return Status::ok(); }
  Status record(hal::Event&) override { return Status::ok(); }
  Status wait(const hal::Event&) override { return Status::ok(); }
  void* native_handle() override { return nullptr; }
};

class CpuEvent final : public hal::Event {
 public:
  bool query() const override { return true; }
  Status synchronize() override { return Status::ok(); }
};

class CpuAllocator final : public hal::Allocator {
 public:
  Result<void*> allocate(size_t bytes, size_t alignment) override {
    if (bytes == 0 || alignment == 0 || (alignment & (alignment - 1)) != 0)
      return Status::make(ErrorCode::kInvalidArgument, "CpuAllocator: bad size or alignment");
    const size_t a = alignment < 64 ? 64 : alignment;
    void* p = std::aligned_alloc(a, (bytes + a - 1) / a * a);
    if (p == nullptr) return Status::make(ErrorCode::kOutOfMemory, "CpuAllocator: out of memory");
    return p;
  }
  void deallocate(void* p) override { std::free(p); }
};

class CpuExecutable final : public hal::Executable {
 public:
  CpuExecutable(ops::ExecutablePlan plan, hal::Allocator& a) : plan_(std::move(plan)), alloc_(&a) {
    for (const auto& t : plan_.input_types) in_.push_back({t.dtype, t.shape});
    for (const auto& t : plan_.output_types) out_.push_back({t.dtype, t.shape});
  }
  Status run(std::span<const Tensor> inputs, std::span<Tensor> outputs, hal::Stream& stream) override {
    FRAME_RETURN_IF_ERROR(hal::validate_io_signature(inputs, in_, "CpuExecutable::run: input"));
    FRAME_RETURN_IF_ERROR(hal::validate_io_signature(outputs, out_, "CpuExecutable::run: output"));
    std::shared_ptr<Storage> arena;
    if (plan_.arena_total_bytes > 0) {
      auto st = Storage::allocate(*alloc_, plan_.arena_total_bytes, kDefaultAlignment, cpu_device());
      if (!st.is_ok()) return st.status();
      arena = st.value();
    }
    std::vector<Tensor> slots(static_cast<size_t>(plan_.slot_count));
    for (size_t i = 0; i < inputs.size(); ++i) slots[i] = inputs[i];
    for (const auto& s : plan_.steps) {
      std::vector<Tensor> ins, outs;
      for (int32_t k : s.input_slots) ins.push_back(slots[static_cast<size_t>(k)]);
      for (size_t j = 0; j < s.output_types.size(); ++j) {
        const auto& t = s.output_types[j];
        if (s.output_arena_offsets[j].has_value() && t.shape.numel() > 0) {
          outs.push_back(Tensor::from_storage_slice(arena, *s.output_arena_offsets[j], t.shape, t.dtype, cpu_device()));
        } else {
          auto e = Tensor::empty(t.shape, t.dtype, cpu_device(), *alloc_);
          if (!e.is_ok()) return e.status();
          outs.push_back(e.value());
        }
      }
      ops::KernelContext ctx{ins, outs, &s.attrs, cpu_device(), &stream, nullptr};
      Status st = s.kernel(ctx);
      if (!st.is_ok()) return Status::make(st.code(), "CpuExecutable::run: op '" + s.op + "' kernel failed: " + std::string(st.message()));
      for (size_t j = 0; j < s.output_slots.size(); ++j) slots[static_cast<size_t>(s.output_slots[j])] = outs[j];
    }
    for (size_t i = 0; i < plan_.output_slots.size(); ++i) {
      const Tensor& src = slots[static_cast<size_t>(plan_.output_slots[i])];
      const size_t bytes = static_cast<size_t>(src.numel()) * src.dtype().itemsize();
      if (bytes) std::memmove(outputs[i].raw_data(), src.raw_data(), bytes);
    }
    return Status::ok();
  }
  std::vector<hal::IoSpec> input_signature() const override { return in_; }
  std::vector<hal::IoSpec> output_signature() const override { return out_; }

 private:
  ops::ExecutablePlan plan_;
  hal::Allocator* alloc_;
  std::vector<hal::IoSpec> in_, out_;
};

class CpuBackend final : public hal::Backend {
 public:
  std::string_view name() const override { return kCpuBackendName; }
  Result<int32_t> device_count() const override { return 1; }
  Result<std::unique_ptr<hal::Stream>> create_stream(Device) override {
    return std::unique_ptr<hal::Stream>(std::make_unique<CpuStream>());
  }
  Result<std::unique_ptr<hal::Event>> create_event(Device) override {
    return std::unique_ptr<hal::Event>(std::make_unique<CpuEvent>());
  }
  hal::Allocator* allocator(Device d) override { return d.backend == kCpuBackendName && d.index == 0 ? &alloc_ : nullptr; }
  Status copy(void* dst, Device, const void* src, Device, size_t bytes, hal::Stream*) override {
    if (bytes) std::memmove(dst, src, bytes);
    return Status::ok();
  }
  Result<std::unique_ptr<hal::Executable>> compile(const ir::Graph& g, const hal::CompileOptions&) override {
    auto plan = ops::build_executable_plan(g, kCpuBackendName);
    if (!plan.is_ok()) return plan.status();
    return std::unique_ptr<hal::Executable>(std::make_unique<CpuExecutable>(std::move(plan.value()), alloc_));
  }
  Status launch(const hal::KernelInvocation& inv, hal::Stream* stream) override {
    auto k = ops::KernelRegistry::instance().find(inv.op, kCpuBackendName);
    if (!k.is_ok()) return Status::make(ErrorCode::kUnimplemented, std::string(k.status().message()));
    ops::KernelContext ctx{inv.inputs, inv.outputs, inv.attrs, inv.device, stream, nullptr};
    return k.value()(ctx);
  }

 private:
  CpuAllocator alloc_;
};

// ---- kernels over cpu_kernels.cpp -------------------------------------------------------------------------

int dcode(DType d) { return static_cast<int>(d.code()); }
Status rc(int r, const char* op) {
  return r == 0 ? Status::ok() : Status::make(ErrorCode::kInvalidArgument, std::string("oracle cpu kernel '") + op + "' rejected its arguments");
}
template <typename T>
const T* attr(const ops::KernelContext& c, const char* n) {
  auto it = c.attrs->find(n);
  return it == c.attrs->end() ? nullptr : std::get_if<T>(&it->second);
}

Status ew(ops::KernelContext& c, std::vector<uint8_t> ops, std::vector<int8_t> ar) {
  std::vector<const void*> ins;
  for (const Tensor& t : c.inputs) ins.push_back(t.raw_data());
  return rc(oracle_ew_program(dcode(c.outputs[0].dtype()), static_cast<int>(ops.size()), ops.data(), ar.data(), ins.data(),
                              static_cast<int>(ins.size()), c.outputs[0].raw_data(), c.outputs[0].numel()),
            "elementwise");
}
template <uint8_t Op, int Ar>
Status ew_kernel(ops::KernelContext& c) {
  return ew(c, {Op}, {static_cast<int8_t>(Ar)});
}
Status fused_kernel(ops::KernelContext& c) {
  ops::FusedElementwiseChain ch;
  FRAME_RETURN_IF_ERROR(ops::decode_and_validate_fused_chain(*c.attrs, static_cast<int64_t>(c.inputs.size()), ch));
  std::vector<uint8_t> codes;
  std::vector<int8_t> ar;
  for (size_t i = 0; i < ch.sub_ops.size(); ++i) {
    const std::string& s = ch.sub_ops[i];
    codes.push_back(s == "add" ? 1 : s == "mul" ? 2 : s == "relu" ? 3 : s == "square" ? 4 : s == "gelu" ? 5 : 0);
    ar.push_back(static_cast<int8_t>(ch.arities[i]));
  }
  return ew(c, codes, ar);
}
Status matmul_kernel(ops::KernelContext& c) {
  const auto& a = c.inputs[0].shape();
  return rc(oracle_matmul(dcode(c.outputs[0].dtype()), c.inputs[0].raw_data(), c.inputs[1].raw_data(),
                          c.outputs[0].raw_data(), a.dim(0), c.inputs[1].shape().dim(1), a.dim(1)),
            "matmul");
}
Status conv_kernel(ops::KernelContext& c) {
  const auto& x = c.inputs[0].shape();
  const auto& w = c.inputs[1].shape();
  const auto* s = attr<std::vector<int64_t>>(c, "stride");
  const auto* p = attr<std::vector<int64_t>>(c, "padding");
  const auto* g = attr<int64_t>(c, "groups");
  const int64_t geom[12] = {x.dim(0), x.dim(1), x.dim(2), x.dim(3), w.dim(0), w.dim(2), w.dim(3), (*s)[0], (*s)[1], (*p)[0], (*p)[1], *g};
  return rc(oracle_conv2d(dcode(c.outputs[0].dtype()), c.inputs[0].raw_data(), c.inputs[1].raw_data(),
                          c.inputs.size() == 3 ? c.inputs[2].raw_data() : nullptr, c.outputs[0].raw_data(), geom),
            "conv2d");
}
Status softmax_kernel(ops::KernelContext& c) {
  const auto& x = c.inputs[0].shape();
  return rc(oracle_softmax(dcode(c.outputs[0].dtype()), c.inputs[0].raw_data(), c.outputs[0].raw_data(), x.dim(0), x.dim(1)), "softmax");
}
Status layer_norm_kernel(ops::KernelContext& c) {
  const auto& x = c.inputs[0].shape();
  return rc(oracle_layer_norm(dcode(c.outputs[0].dtype()), c.inputs[0].raw_data(), c.inputs[1].raw_data(), c.inputs[2].raw_data(),
                              c.outputs[0].raw_data(), x.dim(0), x.dim(1), *attr<double>(c, "eps")),
            "layer_norm");
}
template <int Mode>
Status pool_kernel(ops::KernelContext& c) {
  const auto& x = c.inputs[0].shape();
  const auto* k = attr<std::vector<int64_t>>(c, "kernel");
  const auto* s = attr<std::vector<int64_t>>(c, "stride");
  const auto* p = attr<std::vector<int64_t>>(c, "padding");
  const int64_t geom[10] = {x.dim(0), x.dim(1), x.dim(2), x.dim(3), (*k)[0], (*k)[1], (*s)[0], (*s)[1], (*p)[0], (*p)[1]};
  return rc(oracle_pool2d(dcode(c.outputs[0].dtype()), Mode, c.inputs[0].raw_data(), c.outputs[0].raw_data(), geom), "pool2d");
}
Status reshape_kernel(ops::KernelContext& c) {
  std::memmove(c.outputs[0].raw_data(), c.inputs[0].raw_data(), static_cast<size_t>(c.inputs[0].numel()) * c.inputs[0].dtype().itemsize());
  return Status::ok();
}
Status transpose_kernel(ops::KernelContext& c) {
  const auto& x = c.inputs[0].shape();
  return rc(oracle_transpose(static_cast<int>(c.inputs[0].dtype().itemsize()), c.inputs[0].raw_data(), c.outputs[0].raw_data(),
                             static_cast<int>(x.rank()), x.dims().data(), attr<std::vector<int64_t>>(c, "perm")->data()),
            "transpose");
}
Status slice_kernel(ops::KernelContext& c) {
  const auto& x = c.inputs[0].shape();
  return rc(oracle_slice(static_cast<int>(c.inputs[0].dtype().itemsize()), c.inputs[0].raw_data(), c.outputs[0].raw_data(),
                         static_cast<int>(x.rank()), x.dims().data(), *attr<int64_t>(c, "axis"), *attr<int64_t>(c, "start"),
                         *attr<int64_t>(c, "stop")),
            "slice");
}
Status concat_kernel(ops::KernelContext& c) {
  std::vector<const void*> xs;
  std::vector<int64_t> dims;
  for (const Tensor& t : c.inputs) {
    xs.push_back(t.raw_data());
    dims.insert(dims.end(), t.shape().dims().begin(), t.shape().dims().end());
  }
  return rc(oracle_concat(static_cast<int>(c.outputs[0].dtype().itemsize()), xs.data(), static_cast<int>(xs.size()),
                          c.outputs[0].raw_data(), static_cast<int>(c.outputs[0].shape().rank()), dims.data(),
                          *attr<int64_t>(c, "axis")),
            "concat");
}
Status constant_kernel(ops::KernelContext& c) { return ops::fill_tensor_from_constant_attrs(*c.attrs, c.outputs[0]); }

// ---- training path ----
template <int Rhs>
Status matmul_grad_kernel(ops::KernelContext& c) {
  const auto& p = c.inputs[0].shape();
  const auto& q = c.inputs[1].shape();
  // lhs: gy [m,n], b [k,n]; rhs: a [m,k], gy [m,n]
  const int64_t m = p.dim(0), n = Rhs ? q.dim(1) : p.dim(1), k = Rhs ? p.dim(1) : q.dim(0);
  return rc(oracle_matmul_grad(dcode(c.outputs[0].dtype()), Rhs, c.inputs[0].raw_data(), c.inputs[1].raw_data(),
                               c.outputs[0].raw_data(), m, n, k),
            "matmul_grad");
}
template <int Filter>
Status conv_grad_kernel(ops::KernelContext& c) {
  // input grad: (dy, w) -> dx of input_shape; filter grad: (x, dy) -> dw of filter_shape
  const Shape x = Filter ? c.inputs[0].shape() : *attr<Shape>(c, "input_shape");
  const Shape w = Filter ? *attr<Shape>(c, "filter_shape") : c.inputs[1].shape();
  const auto* s = attr<std::vector<int64_t>>(c, "stride");
  const auto* p = attr<std::vector<int64_t>>(c, "padding");
  const auto* g = attr<int64_t>(c, "groups");
  const int64_t geom[12] = {x.dim(0), x.dim(1), x.dim(2), x.dim(3), w.dim(0), w.dim(2), w.dim(3), (*s)[0], (*s)[1], (*p)[0], (*p)[1], *g};
  const int dt = dcode(c.outputs[0].dtype());
  if (Filter)
    return rc(oracle_conv2d_grad_filter(dt, c.inputs[0].raw_data(), c.inputs[1].raw_data(), c.outputs[0].raw_data(), geom), "conv2d_grad_filter");
  return rc(oracle_conv2d_grad_input(dt, c.inputs[0].raw_data(), c.inputs[1].raw_data(), c.outputs[0].raw_data(), geom), "conv2d_grad_input");
}
template <int Mode>
Status pool_grad_kernel(ops::KernelContext& c) {
  const Shape x = *attr<Shape>(c, "input_shape");
  const auto* k = attr<std::vector<int64_t>>(c, "kernel");
  const auto* s = attr<std::vector<int64_t>>(c, "stride");
  const auto* p = attr<std::vector<int64_t>>(c, "padding");
  const int64_t geom[10] = {x.dim(0), x.dim(1), x.dim(2), x.dim(3), (*k)[0], (*k)[1], (*s)[0], (*s)[1], (*p)[0], (*p)[1]};
  return rc(oracle_pool2d_grad(dcode(c.outputs[0].dtype()), Mode, c.inputs[0].raw_data(),
                               Mode == 0 ? c.inputs[1].raw_data() : nullptr, c.outputs[0].raw_data(), geom),
            "pool2d_grad");
}
std::vector<uint8_t> reduced_mask(const Shape& x, const std::vector<int64_t>& axes) {
  std::vector<uint8_t> r(static_cast<size_t>(x.rank()), axes.empty() ? 1 : 0);
  for (int64_t a : axes) r[static_cast<size_t>(a)] = 1;
  return r;
}
Status sum_kernel(ops::KernelContext& c) {
  const Shape& x = c.inputs[0].shape();
  const auto mask = reduced_mask(x, *attr<std::vector<int64_t>>(c, "axes"));
  return rc(oracle_sum(dcode(c.outputs[0].dtype()), c.inputs[0].raw_data(), c.outputs[0].raw_data(), static_cast<int>(x.rank()),
                       x.dims().data(), mask.data()),
            "sum");
}
Status sum_grad_kernel(ops::KernelContext& c) {
  const Shape x = *attr<Shape>(c, "input_shape");
  const auto mask = reduced_mask(x, *attr<std::vector<int64_t>>(c, "axes"));
  return rc(oracle_sum_grad(static_cast<int>(c.outputs[0].dtype().itemsize()), c.inputs[0].raw_data(), c.outputs[0].raw_data(),
                            static_cast<int>(x.rank()), x.dims().data(), mask.data()),
            "sum_grad");
}
Status mse_loss_kernel(ops::KernelContext& c) {
  return rc(oracle_mse_loss(dcode(c.outputs[0].dtype()), c.inputs[0].raw_data(), c.inputs[1].raw_data(), c.outputs[0].raw_data(),
                            c.inputs[0].numel()),
            "mse_loss");
}
Status mse_loss_grad_kernel(ops::KernelContext& c) {
  return rc(oracle_mse_loss_grad(dcode(c.outputs[0].dtype()), c.inputs[0].raw_data(), c.inputs[1].raw_data(), c.inputs[2].raw_data(),
                                 c.outputs[0].raw_data(), c.inputs[0].numel()),
            "mse_loss_grad");
}

}  // namespace oracle_cpu

FRAME_REGISTER_BACKEND(frame::kCpuBackendName, oracle_cpu::CpuBackend);
FRAME_REGISTER_KERNEL("add", frame::kCpuBackendName, (&oracle_cpu::ew_kernel<1, 2>));
FRAME_REGISTER_KERNEL("mul", frame::kCpuBackendName, (&oracle_cpu::ew_kernel<2, 2>));
FRAME_REGISTER_KERNEL("relu", frame::kCpuBackendName, (&oracle_cpu::ew_kernel<3, 1>));
FRAME_REGISTER_KERNEL("square", frame::kCpuBackendName, (&oracle_cpu::ew_kernel<4, 1>));
FRAME_REGISTER_KERNEL("gelu", frame::kCpuBackendName, (&oracle_cpu::ew_kernel<5, 1>));
FRAME_REGISTER_KERNEL(frame::ops::kFusedElementwiseOpName, frame::kCpuBackendName, &oracle_cpu::fused_kernel);
FRAME_REGISTER_KERNEL("matmul", frame::kCpuBackendName, &oracle_cpu::matmul_kernel);
FRAME_REGISTER_KERNEL("conv2d", frame::kCpuBackendName, &oracle_cpu::conv_kernel);
FRAME_REGISTER_KERNEL("softmax", frame::kCpuBackendName, &oracle_cpu::softmax_kernel);
FRAME_REGISTER_KERNEL("layer_norm", frame::kCpuBackendName, &oracle_cpu::layer_norm_kernel);
FRAME_REGISTER_KERNEL("max_pool2d", frame::kCpuBackendName, &oracle_cpu::pool_kernel<0>);
FRAME_REGISTER_KERNEL("avg_pool2d", frame::kCpuBackendName, &oracle_cpu::pool_kernel<1>);
FRAME_REGISTER_KERNEL("reshape", frame::kCpuBackendName, &oracle_cpu::reshape_kernel);
FRAME_REGISTER_KERNEL("transpose", frame::kCpuBackendName, &oracle_cpu::transpose_kernel);
FRAME_REGISTER_KERNEL("slice", frame::kCpuBackendName, &oracle_cpu::slice_kernel);
FRAME_REGISTER_KERNEL("concat", frame::kCpuBackendName, &oracle_cpu::concat_kernel);
FRAME_REGISTER_KERNEL(frame::ops::kConstantOpName, frame::kCpuBackendName, &oracle_cpu::constant_kernel);
FRAME_REGISTER_KERNEL("relu_grad_internal", frame::kCpuBackendName, (&oracle_cpu::ew_kernel<6, 2>));
FRAME_REGISTER_KERNEL("sigmoid", frame::kCpuBackendName, (&oracle_cpu::ew_kernel<7, 1>));
FRAME_REGISTER_KERNEL("tanh", frame::kCpuBackendName, (&oracle_cpu::ew_kernel<8, 1>));
FRAME_REGISTER_KERNEL("rsqrt", frame::kCpuBackendName, (&oracle_cpu::ew_kernel<9, 1>));
FRAME_REGISTER_KERNEL("gelu_grad_internal", frame::kCpuBackendName, (&oracle_cpu::ew_kernel<10, 2>));
FRAME_REGISTER_KERNEL("matmul_grad_lhs_internal", frame::kCpuBackendName, &oracle_cpu::matmul_grad_kernel<0>);
FRAME_REGISTER_KERNEL("matmul_grad_rhs_internal", frame::kCpuBackendName, &oracle_cpu::matmul_grad_kernel<1>);
FRAME_REGISTER_KERNEL("conv2d_grad_input_internal", frame::kCpuBackendName, &oracle_cpu::conv_grad_kernel<0>);
FRAME_REGISTER_KERNEL("conv2d_grad_filter_internal", frame::kCpuBackendName, &oracle_cpu::conv_grad_kernel<1>);
FRAME_REGISTER_KERNEL("max_pool2d_grad_internal", frame::kCpuBackendName, &oracle_cpu::pool_grad_kernel<0>);
FRAME_REGISTER_KERNEL("avg_pool2d_grad_internal", frame::kCpuBackendName, &oracle_cpu::pool_grad_kernel<1>);
FRAME_REGISTER_KERNEL("sum", frame::kCpuBackendName, &oracle_cpu::sum_kernel);
FRAME_REGISTER_KERNEL("sum_grad_internal", frame::kCpuBackendName, &oracle_cpu::sum_grad_kernel);
FRAME_REGISTER_KERNEL("mse_loss", frame::kCpuBackendName, &oracle_cpu::mse_loss_kernel);
FRAME_REGISTER_KERNEL("mse_loss_grad_internal", frame::kCpuBackendName, &oracle_cpu::mse_loss_grad_kernel);

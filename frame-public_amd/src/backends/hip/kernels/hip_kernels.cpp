// KernelFn wrappers of the `hip` backend: argument checks on the host, then one enqueue through the C ABI of
// libframe_hip_kernels.so on the context's stream. Registered with FRAME_REGISTER_KERNEL(op, "hip", fn) like
// every Frame backend's kernels (reference: include/frame/ops/kernel_registry.h:104-107). The design analogs
// replaced are the cuda kernels under src/backends/cuda/kernels/ (cuBLASLt, cuDNN and the .cu files).
#include <algorithm>
#include <array>
#include <cstdint>
#include <string>
#include <vector>

#include <frame/core/tensor.h>
#include <frame/hal/backend.h>
#include <frame/ops/constant_utils.h>
#include <frame/ops/fused_elementwise_utils.h>
#include <frame/ops/kernel_registry.h>

#include "../hip_backend.h"

namespace frame::backends::hip {
namespace {

using ops::KernelContext;

Status invalid(const std::string& op, const std::string& msg) {
  return Status::make(ErrorCode::kInvalidArgument, "op '" + op + "' (hip): " + msg);
}

// fh dtype code of a floating-point tensor, or an kUnimplemented status.
Result<int32_t> float_code(const std::string& op, DType d) {
  switch (d.code()) {
    case DTypeCode::kFloat32: return static_cast<int32_t>(FH_F32);
    case DTypeCode::kFloat16: return static_cast<int32_t>(FH_F16);
    case DTypeCode::kBFloat16: return static_cast<int32_t>(FH_BF16);
    default:
      return Status::make(ErrorCode::kUnimplemented,
                          "op '" + op + "' on backend 'hip' does not support dtype '" + std::string(d.name()) + "'");
  }
}

Status arity(const KernelContext& ctx, const std::string& op, size_t n_in, size_t n_out) {
  if (ctx.inputs.size() != n_in) return invalid(op, "expects " + std::to_string(n_in) + " input(s), got " + std::to_string(ctx.inputs.size()));
  if (ctx.outputs.size() != n_out) return invalid(op, "expects " + std::to_string(n_out) + " output(s), got " + std::to_string(ctx.outputs.size()));
  return Status::ok();
}

// Element-type comparisons and sizes for the argument checks below.
bool same_elem_type(const Tensor& a, const Tensor& b) { return a.dtype() == b.dtype(); }
bool same_elem_type(const Tensor& a, DType b) { return a.dtype() == b; }
size_t elem_bytes(const Tensor& t) { return t.dtype().itemsize(); }

Status same_dtype(const KernelContext& ctx, const std::string& op) {
  const DType d = ctx.outputs[0].dtype();
  for (const Tensor& t : ctx.inputs)
    if (!same_elem_type(t, d))
      return invalid(op, "input dtype '" + std::string(t.dtype().name()) + "' differs from output dtype '" + std::string(d.name()) + "'");
  return Status::ok();
}

template <typename T>
const T* attr(const KernelContext& ctx, const char* name) {
  if (ctx.attrs == nullptr) return nullptr;
  auto it = ctx.attrs->find(name);
  return it == ctx.attrs->end() ? nullptr : std::get_if<T>(&it->second);
}

// ---- elementwise ------------------------------------------------------------------------------------------

Status run_program(const KernelContext& ctx, const std::string& op, const std::vector<uint8_t>& codes,
                   const std::vector<int8_t>& arities) {
  FRAME_RETURN_IF_ERROR(same_dtype(ctx, op));
  Result<int32_t> dt = float_code(op, ctx.outputs[0].dtype());
  if (!dt.is_ok()) return dt.status();
  const int64_t n = ctx.outputs[0].numel();
  std::vector<const void*> ins;
  for (const Tensor& t : ctx.inputs) {
    if (t.numel() != n) return invalid(op, "operand element count " + std::to_string(t.numel()) + " differs from output " + std::to_string(n));
    ins.push_back(t.raw_data());
  }
  FRAME_HIP_RETURN_IF_ERROR(fh_ew_program(dt.value(), static_cast<int32_t>(codes.size()), codes.data(), arities.data(),
                                          ins.data(), static_cast<int32_t>(ins.size()), ctx.outputs[0].raw_data(), n,
                                          /*round_between=*/1, stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

template <uint8_t Code, int Arity>
Status ew_kernel(KernelContext& ctx) {
  static const std::string names[] = {"",        "add",  "mul",   "relu", "square", "gelu", "relu_grad_internal",
                                      "sigmoid", "tanh", "rsqrt", "gelu_grad_internal"};
  const std::string& op = names[Code];
  FRAME_RETURN_IF_ERROR(arity(ctx, op, Arity, 1));
  return run_program(ctx, op, {Code}, {static_cast<int8_t>(Arity)});
}

Status fused_kernel(KernelContext& ctx) {
  const std::string op(ops::kFusedElementwiseOpName);
  if (ctx.outputs.size() != 1) return invalid(op, "expects 1 output");
  if (ctx.attrs == nullptr) return invalid(op, "requires attrs");
  ops::FusedElementwiseChain chain;
  FRAME_RETURN_IF_ERROR(ops::decode_and_validate_fused_chain(*ctx.attrs, static_cast<int64_t>(ctx.inputs.size()), chain));
  if (chain.sub_ops.size() > FH_MAX_SEGMENTS || ctx.inputs.size() > FH_MAX_EW_INPUTS)
    return Status::make(ErrorCode::kUnimplemented, "op '" + op + "' (hip): chain longer than " + std::to_string(FH_MAX_SEGMENTS) + " segments");
  std::vector<uint8_t> codes;
  std::vector<int8_t> ar;
  for (size_t i = 0; i < chain.sub_ops.size(); ++i) {
    const uint8_t c = ew_code(chain.sub_ops[i]);
    if (c == 0)
      return Status::make(ErrorCode::kUnimplemented, "op '" + op + "' (hip): sub-op '" + chain.sub_ops[i] + "' has no device kernel");
    codes.push_back(c);
    ar.push_back(static_cast<int8_t>(chain.arities[i]));
  }
  return run_program(ctx, op, codes, ar);
}

Status ew_program_kernel(KernelContext& ctx) {
  const std::string op(kEwProgramOp);
  if (ctx.outputs.size() != 1) return invalid(op, "expects 1 output");
  const auto* prog = attr<std::vector<int64_t>>(ctx, "ew_ops");
  if (prog == nullptr || prog->empty() || prog->size() > FH_MAX_SEGMENTS) return invalid(op, "missing or malformed ew_ops");
  std::vector<uint8_t> codes;
  std::vector<int8_t> ar;
  size_t need = 0;
  for (size_t i = 0; i < prog->size(); ++i) {
    const int64_t c = (*prog)[i];
    if (c < FH_EW_ADD || c > FH_EW_RELU_MASK) return invalid(op, "unknown op code " + std::to_string(c));
    const bool binary = c == FH_EW_ADD || c == FH_EW_MUL || c == FH_EW_RELU_GRAD || c == FH_EW_GELU_GRAD || c == FH_EW_RELU_MASK;
    codes.push_back(static_cast<uint8_t>(c));
    ar.push_back(binary ? 2 : 1);
    need += i == 0 ? (binary ? 2 : 1) : (binary ? 1 : 0);
  }
  if (ctx.inputs.size() != need) return invalid(op, "expects " + std::to_string(need) + " inputs");
  return run_program(ctx, op, codes, ar);
}

// ---- contractions -----------------------------------------------------------------------------------------

// Epilogue operands are ctx.inputs[first..]; binary segments consume them in order.
Result<fh_epilogue> make_epilogue(const KernelContext& ctx, const std::string& op, size_t first) {
  fh_epilogue ep{};
  const auto* prog = attr<std::vector<int64_t>>(ctx, "ep_ops");
  if (prog == nullptr) return ep;
  if (prog->size() > FH_MAX_SEGMENTS) return invalid(op, "epilogue longer than " + std::to_string(FH_MAX_SEGMENTS) + " segments");
  ep.nseg = static_cast<int32_t>(prog->size());
  ep.round_between = 1;
  size_t next = first;
  const int64_t n = ctx.outputs[0].numel();
  for (size_t s = 0; s < prog->size(); ++s) {
    ep.ops[s] = static_cast<uint8_t>((*prog)[s]);
    if (ep.ops[s] == FH_EW_ADD || ep.ops[s] == FH_EW_MUL) {
      if (next >= ctx.inputs.size()) return invalid(op, "epilogue operand missing");
      const Tensor& t = ctx.inputs[next++];
      if (t.numel() != n || !same_elem_type(t, ctx.outputs[0]))
        return invalid(op, "epilogue operand has the wrong shape or dtype");
      ep.ins[s] = t.raw_data();
    }
  }
  if (next != ctx.inputs.size()) return invalid(op, "unused epilogue operands");
  return ep;
}

Status gemm_impl(KernelContext& ctx, const std::string& op, size_t n_main) {
  if (ctx.inputs.size() < n_main || ctx.outputs.size() != 1) return invalid(op, "bad operand count");
  const Tensor& a = ctx.inputs[0];
  const Tensor& b = ctx.inputs[1];
  Tensor& c = ctx.outputs[0];
  if (a.shape().rank() != 2 || b.shape().rank() != 2 || c.shape().rank() != 2) return invalid(op, "operands must be rank-2");
  const int64_t m = a.shape().dim(0), k = a.shape().dim(1), n = b.shape().dim(1);
  if (b.shape().dim(0) != k || c.shape().dim(0) != m || c.shape().dim(1) != n)
    return invalid(op, "shape mismatch " + a.shape().to_string() + " x " + b.shape().to_string() + " -> " + c.shape().to_string());
  FRAME_RETURN_IF_ERROR(same_dtype(ctx, op));
  Result<int32_t> dt = float_code(op, c.dtype());
  if (!dt.is_ok()) return dt.status();
  Result<fh_epilogue> ep = make_epilogue(ctx, op, n_main);
  if (!ep.is_ok()) return ep.status();
  const auto* any = attr<int64_t>(ctx, "any_order");
  const auto* row_softmax = attr<int64_t>(ctx, "row_softmax");
  const int32_t flags = ((any != nullptr && *any != 0) ? FH_GEMM_ANY_ORDER : 0) |
                        ((row_softmax != nullptr && *row_softmax != 0) ? FH_GEMM_ROW_SOFTMAX : 0);
  FRAME_HIP_RETURN_IF_ERROR(fh_gemm_ex(dt.value(), a.raw_data(), b.raw_data(), c.raw_data(), m, n, k,
                                       ep.value().nseg > 0 ? &ep.value() : nullptr, flags, stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

// kGemmGroupedOp: inputs [A, B_0 .. B_{g-1}, epilogue operands group by group], outputs C_0 .. C_{g-1}.
Status gemm_grouped_kernel(KernelContext& ctx) {
  const std::string op(kGemmGroupedOp);
  const auto* groups_attr = attr<int64_t>(ctx, "groups");
  if (groups_attr == nullptr || *groups_attr < 1 || *groups_attr > FH_GEMM_MAX_GROUPS) return invalid(op, "bad groups attribute");
  const size_t g = static_cast<size_t>(*groups_attr);
  if (ctx.outputs.size() != g || ctx.inputs.size() < 1 + g) return invalid(op, "bad operand count");
  const Tensor& a = ctx.inputs[0];
  if (a.shape().rank() != 2) return invalid(op, "A must be rank-2");
  const int64_t m = a.shape().dim(0), k = a.shape().dim(1);
  const Tensor& b0 = ctx.inputs[1];
  if (b0.shape().rank() != 2 || b0.shape().dim(0) != k) return invalid(op, "B shape mismatch");
  const int64_t n = b0.shape().dim(1);
  FRAME_RETURN_IF_ERROR(same_dtype(ctx, op));
  Result<int32_t> dt = float_code(op, a.dtype());
  if (!dt.is_ok()) return dt.status();
  const auto* prog = attr<std::vector<int64_t>>(ctx, "ep_ops");
  size_t binary = 0;
  if (prog != nullptr) {
    if (prog->size() > FH_MAX_SEGMENTS) return invalid(op, "epilogue longer than " + std::to_string(FH_MAX_SEGMENTS) + " segments");
    for (int64_t c : *prog) binary += (c == FH_EW_ADD || c == FH_EW_MUL) ? 1 : 0;
  }
  if (ctx.inputs.size() != 1 + g + g * binary) return invalid(op, "epilogue operand count does not match the program");
  std::vector<const void*> bs(g);
  std::vector<void*> cs(g);
  std::vector<fh_epilogue> eps(g);
  size_t next = 1 + g;
  for (size_t i = 0; i < g; ++i) {
    const Tensor& b = ctx.inputs[1 + i];
    Tensor& c = ctx.outputs[i];
    if (b.shape().rank() != 2 || b.shape().dim(0) != k || b.shape().dim(1) != n || c.shape().rank() != 2 ||
        c.shape().dim(0) != m || c.shape().dim(1) != n)
      return invalid(op, "group " + std::to_string(i) + ": shape mismatch");
    bs[i] = b.raw_data();
    cs[i] = c.raw_data();
    eps[i] = fh_epilogue{};
    if (prog != nullptr) {
      eps[i].nseg = static_cast<int32_t>(prog->size());
      eps[i].round_between = 1;
      for (size_t s = 0; s < prog->size(); ++s) {
        eps[i].ops[s] = static_cast<uint8_t>((*prog)[s]);
        if (eps[i].ops[s] == FH_EW_ADD || eps[i].ops[s] == FH_EW_MUL) {
          const Tensor& t = ctx.inputs[next++];
          if (t.numel() != m * n || !same_elem_type(t, c))
            return invalid(op, "epilogue operand has the wrong shape or dtype");
          eps[i].ins[s] = t.raw_data();
        }
      }
    }
  }
  const auto* any = attr<int64_t>(ctx, "any_order");
  const int32_t flags = (any != nullptr && *any != 0) ? FH_GEMM_ANY_ORDER : 0;
  FRAME_HIP_RETURN_IF_ERROR(fh_gemm_grouped(dt.value(), a.raw_data(), static_cast<int32_t>(g), bs.data(), cs.data(), m, n,
                                            k, eps.data(), flags, stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

Status matmul_kernel(KernelContext& ctx) {
  FRAME_RETURN_IF_ERROR(arity(ctx, "matmul", 2, 1));
  return gemm_impl(ctx, "matmul", 2);
}

Status gemm_epilogue_kernel(KernelContext& ctx) {
  const auto* n_main = attr<int64_t>(ctx, "n_main_inputs");
  return gemm_impl(ctx, std::string(kGemmEpilogueOp), n_main ? static_cast<size_t>(*n_main) : 2);
}

// An NCHW conv2d (an eager Backend::launch, or a node HipBackend::compile did not lower) whose geometry the
// implicit-GEMM kernel accepts runs on MFMA: channels-last copies of x and w (or their C8 packs when Cin <= 8,
// 16-bit) go to device temporaries from the backend's allocator, then the MFMA conv writes y NCHW with the bias
// and epilogue. The temporaries go back to the allocator when this call returns; it hands them out again only
// after the device has gone idle, so the queued kernels still own them. Returns false when the geometry is
// outside that kernel's envelope (the caller then runs the direct kernel).
Result<bool> conv_via_channels_last(const KernelContext& ctx, const std::string& op, int32_t dt, const int64_t geom[12],
                                    const Tensor* bias, const fh_epilogue& ep) {
  const Tensor& x = ctx.inputs[0];
  const Tensor& w = ctx.inputs[1];
  const bool c8 = dt != FH_F32 && geom[1] <= 8 && geom[11] == 1;
  int64_t g[12];
  std::copy(geom, geom + 12, g);
  if (c8) g[1] = 8;
  if (fh_conv2d_nhwc_supported(dt, g) == 0) return false;
  Result<hal::Backend*> be = hal::BackendRegistry::instance().get(kHipBackendName);
  if (!be.is_ok()) return be.status();
  hal::Allocator* alloc = be.value()->allocator(ctx.device);
  if (alloc == nullptr) return Status::make(ErrorCode::kInternal, "op '" + op + "' (hip): no allocator for the device");
  const int64_t n = geom[0], cin = geom[1], h = geom[2], wd = geom[3], cout = geom[4], kh = geom[5], kw = geom[6];
  // the resident-patch kernel reads NCHW activations itself where the geometry allows; otherwise a channels-last copy
  const bool nchw_in = !c8 && fh_conv2d_nchw_in_supported(dt, g) != 0;
  Result<Tensor> xt = Tensor::empty(nchw_in ? Shape({1}) : Shape({n, h, wd, c8 ? 8 : cin}), x.dtype(), ctx.device, *alloc);
  if (!xt.is_ok()) return xt.status();
  Result<Tensor> wt = c8 ? Tensor::empty(Shape({cout, fh_conv_c8_filter_k(kh, kw)}), w.dtype(), ctx.device, *alloc)
                         : Tensor::empty(Shape({cout, kh, kw, cin}), w.dtype(), ctx.device, *alloc);
  if (!wt.is_ok()) return wt.status();
  void* s = stream_handle(ctx);
  const std::string what = "op '" + op + "' (hip)";
  if (c8) {
    FRAME_HIP_RETURN_IF_ERROR(fh_conv_pack_input_c8(x.raw_data(), xt.value().raw_data(), n, static_cast<int32_t>(cin), h * wd, s), what);
    FRAME_HIP_RETURN_IF_ERROR(fh_conv_pack_filter_c8(w.raw_data(), wt.value().raw_data(), static_cast<int32_t>(cout),
                                                     static_cast<int32_t>(cin), static_cast<int32_t>(kh),
                                                     static_cast<int32_t>(kw), s), what);
  } else {
    const int32_t es = static_cast<int32_t>(x.dtype().itemsize());
    if (!nchw_in)
      FRAME_HIP_RETURN_IF_ERROR(fh_transpose_batched(es, x.raw_data(), xt.value().raw_data(), n, cin, h * wd, s), what);
    FRAME_HIP_RETURN_IF_ERROR(fh_transpose_batched(es, w.raw_data(), wt.value().raw_data(), cout, cin, kh * kw, s), what);
  }
  FRAME_HIP_RETURN_IF_ERROR(fh_conv2d_nhwc_fwd_ex(dt, nchw_in ? x.raw_data() : xt.value().raw_data(), wt.value().raw_data(),
                                                  bias ? bias->raw_data() : nullptr, ctx.outputs[0].raw_data(), g,
                                                  ep.nseg > 0 ? &ep : nullptr, nchw_in ? FH_CONV_IN_NCHW : 0, s), what);
  return true;
}

Status conv_impl(KernelContext& ctx, const std::string& op, size_t n_main) {
  if (ctx.inputs.size() < n_main || n_main < 2 || n_main > 3 || ctx.outputs.size() != 1) return invalid(op, "bad operand count");
  const Tensor& x = ctx.inputs[0];
  const Tensor& w = ctx.inputs[1];
  const Tensor* bias = n_main == 3 ? &ctx.inputs[2] : nullptr;
  Tensor& y = ctx.outputs[0];
  const auto* stride = attr<std::vector<int64_t>>(ctx, "stride");
  const auto* pad = attr<std::vector<int64_t>>(ctx, "padding");
  const auto* groups = attr<int64_t>(ctx, "groups");
  if (stride == nullptr || pad == nullptr || groups == nullptr || stride->size() != 2 || pad->size() != 2)
    return invalid(op, "missing or malformed stride/padding/groups attributes");
  if (x.shape().rank() != 4 || w.shape().rank() != 4 || y.shape().rank() != 4) return invalid(op, "operands must be rank-4");
  for (size_t i = 0; i < n_main; ++i)
    if (!same_elem_type(ctx.inputs[i], y))
      return invalid(op, "operand dtypes differ");
  Result<int32_t> dt = float_code(op, y.dtype());
  if (!dt.is_ok()) return dt.status();
  const int64_t geom[12] = {x.shape().dim(0), x.shape().dim(1), x.shape().dim(2), x.shape().dim(3),
                            w.shape().dim(0), w.shape().dim(2), w.shape().dim(3), (*stride)[0],
                            (*stride)[1],     (*pad)[0],        (*pad)[1],        *groups};
  const int64_t oh = (geom[2] + 2 * geom[9] - geom[5]) / geom[7] + 1;
  const int64_t ow = (geom[3] + 2 * geom[10] - geom[6]) / geom[8] + 1;
  if (y.shape() != Shape({geom[0], geom[4], oh, ow})) return invalid(op, "output shape " + y.shape().to_string() + " does not match the geometry");
  if (w.shape().dim(1) * geom[11] != geom[1]) return invalid(op, "filter channels do not match Cin/groups");
  if (bias != nullptr && (bias->shape().rank() != 1 || bias->shape().dim(0) != geom[4])) return invalid(op, "bias must be [Cout]");
  Result<fh_epilogue> ep = make_epilogue(ctx, op, n_main);
  if (!ep.is_ok()) return ep.status();
  if (y.numel() > 0) {
    Result<bool> done = conv_via_channels_last(ctx, op, dt.value(), geom, bias, ep.value());
    if (!done.is_ok()) return done.status();
    if (done.value()) return Status::ok();
  }
  FRAME_HIP_RETURN_IF_ERROR(fh_conv2d_fwd(dt.value(), x.raw_data(), w.raw_data(), bias ? bias->raw_data() : nullptr,
                                          y.raw_data(), geom, ep.value().nseg > 0 ? &ep.value() : nullptr, stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

// x_nhwc [N,H,W,Cin] (or NCHW, in_nchw), w_khwc [Cout,KH,KW,Cin] (or [Cout,Cin,KH,KW], w_oihw), optional bias
// [Cout], then the epilogue operands; y NCHW (or channels-last, out_nhwc). An optional second output is the fp32
// workspace of the split-K form (channels-last output only; fh_conv2d_nhwc_split_workspace sized it).
Status conv_nhwc_kernel(KernelContext& ctx) {
  const std::string op(kConvNhwcOp);
  const auto* n_main_attr = attr<int64_t>(ctx, "n_main_inputs");
  const size_t n_main = n_main_attr ? static_cast<size_t>(*n_main_attr) : 2;
  if (ctx.inputs.size() < n_main || n_main < 2 || n_main > 3 || ctx.outputs.empty() || ctx.outputs.size() > 2)
    return invalid(op, "bad operand count");
  const Tensor& x = ctx.inputs[0];
  const Tensor& w = ctx.inputs[1];
  const Tensor* bias = n_main == 3 ? &ctx.inputs[2] : nullptr;
  Tensor& y = ctx.outputs[0];
  const auto* stride = attr<std::vector<int64_t>>(ctx, "stride");
  const auto* pad = attr<std::vector<int64_t>>(ctx, "padding");
  const auto* groups = attr<int64_t>(ctx, "groups");
  if (stride == nullptr || pad == nullptr || groups == nullptr || stride->size() != 2 || pad->size() != 2)
    return invalid(op, "missing or malformed stride/padding/groups attributes");
  if (x.shape().rank() != 4 || (w.shape().rank() != 4 && w.shape().rank() != 2) || y.shape().rank() != 4)
    return invalid(op, "x and y must be rank-4, the filter rank-4 or rank-2 (C8)");
  for (size_t i = 0; i < n_main; ++i)
    if (!same_elem_type(ctx.inputs[i], y))
      return invalid(op, "operand dtypes differ");
  Result<int32_t> dt = float_code(op, y.dtype());
  if (!dt.is_ok()) return dt.status();
  // filter [Cout,KH,KW,Cin], or the C8 layout [Cout, K8] (Cin == 8) with KH, KW in the filter_hw attribute
  const auto* fhw = attr<std::vector<int64_t>>(ctx, "filter_hw");
  const bool c8 = w.shape().rank() == 2;
  if (c8 && (fhw == nullptr || fhw->size() != 2 || x.shape().dim(3) != 8))
    return invalid(op, "C8 filter needs filter_hw and an input with 8 channels");
  // in_nchw: x is NCHW [N,Cin,H,W] (FH_CONV_IN_NCHW), else channels-last [N,H,W,Cin]; w_oihw: the filter is
  // [Cout,Cin,KH,KW] (FH_CONV_W_OIHW, with in_nchw only)
  const auto* in_nchw_attr = attr<int64_t>(ctx, "in_nchw");
  const bool in_nchw = in_nchw_attr != nullptr && *in_nchw_attr != 0;
  const auto* w_oihw_attr = attr<int64_t>(ctx, "w_oihw");
  const bool w_oihw = w_oihw_attr != nullptr && *w_oihw_attr != 0;
  if (in_nchw && c8) return invalid(op, "NCHW input with the C8 filter");
  if (w_oihw && !in_nchw) return invalid(op, "the [Cout,Cin,KH,KW] filter goes with NCHW input only");
  const int64_t kh = c8 ? (*fhw)[0] : w.shape().dim(w_oihw ? 2 : 1), kw = c8 ? (*fhw)[1] : w.shape().dim(w_oihw ? 3 : 2);
  const int64_t geom[12] = {x.shape().dim(0), x.shape().dim(in_nchw ? 1 : 3), x.shape().dim(in_nchw ? 2 : 1),
                            x.shape().dim(in_nchw ? 3 : 2), w.shape().dim(0), kh, kw, (*stride)[0],
                            (*stride)[1], (*pad)[0], (*pad)[1], *groups};
  if (c8 ? w.shape().dim(1) != fh_conv_c8_filter_k(kh, kw) : w.shape().dim(w_oihw ? 1 : 3) != geom[1])
    return invalid(op, "filter shape does not match the input's channels");
  // 16-bit with 8 input channels is the C8 kernel, which reads the packed [Cout, K8] filter only
  if (!c8 && geom[1] == 8 && dt.value() != FH_F32) return invalid(op, "an 8-channel 16-bit input needs the packed C8 filter");
  const int64_t oh = (geom[2] + 2 * geom[9] - geom[5]) / geom[7] + 1;
  const int64_t ow = (geom[3] + 2 * geom[10] - geom[6]) / geom[8] + 1;
  // out_nhwc: y (and the epilogue operands) channels-last [N,Ho,Wo,Cout], else NCHW
  const auto* out_nhwc_attr = attr<int64_t>(ctx, "out_nhwc");
  const bool out_nhwc = out_nhwc_attr != nullptr && *out_nhwc_attr != 0;
  const Shape want = out_nhwc ? Shape({geom[0], oh, ow, geom[4]}) : Shape({geom[0], geom[4], oh, ow});
  if (y.shape() != want) return invalid(op, "output shape " + y.shape().to_string() + " does not match the geometry");
  if (bias != nullptr && (bias->shape().rank() != 1 || bias->shape().dim(0) != geom[4])) return invalid(op, "bias must be [Cout]");
  Result<fh_epilogue> ep = make_epilogue(ctx, op, n_main);
  if (!ep.is_ok()) return ep.status();
  if (ctx.outputs.size() == 2) {
    Tensor& ws = ctx.outputs[1];
    const bool ws_f32 = same_elem_type(ws, DType::of<float>());
    if (!out_nhwc || in_nchw || c8 || !ws_f32)
      return invalid(op, "the split-K workspace goes with a channels-last output and is float32");
    FRAME_HIP_RETURN_IF_ERROR(fh_conv2d_nhwc_fwd_split(dt.value(), x.raw_data(), w.raw_data(), bias ? bias->raw_data() : nullptr,
                                                       y.raw_data(), geom, ep.value().nseg > 0 ? &ep.value() : nullptr,
                                                       FH_CONV_OUT_NHWC, 0, ws.raw_data(),
                                                       ws.numel() * static_cast<int64_t>(sizeof(float)), stream_handle(ctx)),
                              "op '" + op + "' (hip)");
    return Status::ok();
  }
  FRAME_HIP_RETURN_IF_ERROR(fh_conv2d_nhwc_fwd_ex(dt.value(), x.raw_data(), w.raw_data(), bias ? bias->raw_data() : nullptr,
                                                  y.raw_data(), geom, ep.value().nseg > 0 ? &ep.value() : nullptr,
                                                  (out_nhwc ? FH_CONV_OUT_NHWC : 0) | (in_nchw ? FH_CONV_IN_NCHW : 0) |
                                                      (w_oihw ? FH_CONV_W_OIHW : 0),
                                                  stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

// The stem chain conv2d 7x7/2 + bias [+ relu] + max_pool2d 3x3/2 as one launch (fh_conv2d_stem_pool).
Status conv_stem_pool_kernel(KernelContext& ctx) {
  const std::string op(kConvStemPoolOp);
  if (ctx.inputs.size() < 2 || ctx.inputs.size() > 3 || ctx.outputs.size() != 1)
    return invalid(op, "expects x, w[, bias] and one output");
  const Tensor &x = ctx.inputs[0], &w = ctx.inputs[1];
  Tensor& y = ctx.outputs[0];
  const Tensor* bias = ctx.inputs.size() == 3 ? &ctx.inputs[2] : nullptr;
  const auto* stride = attr<std::vector<int64_t>>(ctx, "stride");
  const auto* pad = attr<std::vector<int64_t>>(ctx, "padding");
  const auto* groups = attr<int64_t>(ctx, "groups");
  const auto* pk = attr<std::vector<int64_t>>(ctx, "kernel");
  const auto* ps = attr<std::vector<int64_t>>(ctx, "pool_stride");
  const auto* pp = attr<std::vector<int64_t>>(ctx, "pool_padding");
  const auto* relu = attr<int64_t>(ctx, "relu");
  if (stride == nullptr || pad == nullptr || groups == nullptr || pk == nullptr || ps == nullptr || pp == nullptr ||
      relu == nullptr || stride->size() != 2 || pad->size() != 2 || pk->size() != 2 || ps->size() != 2 || pp->size() != 2)
    return invalid(op, "missing or malformed attributes");
  if (x.shape().rank() != 4 || w.shape().rank() != 4 || y.shape().rank() != 4) return invalid(op, "x, w and y must be rank-4");
  for (const Tensor& t : ctx.inputs)
    if (!same_elem_type(t, y))
      return invalid(op, "operand dtypes differ");
  Result<int32_t> dt = float_code(op, y.dtype());
  if (!dt.is_ok()) return dt.status();
  const int64_t geom[12] = {x.shape().dim(0), x.shape().dim(1), x.shape().dim(2), x.shape().dim(3), w.shape().dim(0),
                            w.shape().dim(2), w.shape().dim(3), (*stride)[0], (*stride)[1], (*pad)[0], (*pad)[1], *groups};
  const int64_t pool[6] = {(*pk)[0], (*pk)[1], (*ps)[0], (*ps)[1], (*pp)[0], (*pp)[1]};
  if (w.shape().dim(1) != geom[1]) return invalid(op, "filter channels differ from the input's");
  if (bias != nullptr && (bias->shape().rank() != 1 || bias->shape().dim(0) != geom[4])) return invalid(op, "bias must be [Cout]");
  const int64_t oh = (geom[2] + 2 * geom[9] - geom[5]) / geom[7] + 1, ow = (geom[3] + 2 * geom[10] - geom[6]) / geom[8] + 1;
  const int64_t ph = (oh + 2 * pool[4] - pool[0]) / pool[2] + 1, pw = (ow + 2 * pool[5] - pool[1]) / pool[3] + 1;
  if (y.shape() != Shape({geom[0], geom[4], ph, pw})) return invalid(op, "output shape does not match the geometry");
  FRAME_HIP_RETURN_IF_ERROR(fh_conv2d_stem_pool(dt.value(), x.raw_data(), w.raw_data(), bias ? bias->raw_data() : nullptr,
                                                y.raw_data(), geom, pool, *relu != 0 ? 1 : 0, stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

// [d0, d1, d2, d3] -> [d0, d2, d3, d1]
Status channels_last_kernel(KernelContext& ctx) {
  const std::string op(kChannelsLastOp);
  FRAME_RETURN_IF_ERROR(arity(ctx, op, 1, 1));
  const Tensor& x = ctx.inputs[0];
  Tensor& y = ctx.outputs[0];
  if (x.shape().rank() != 4 || !same_elem_type(x, y))
    return invalid(op, "expects a rank-4 input of the output's dtype");
  const Shape& s = x.shape();
  if (y.shape() != Shape({s.dim(0), s.dim(2), s.dim(3), s.dim(1)})) return invalid(op, "output shape does not match [d0,d2,d3,d1]");
  FRAME_HIP_RETURN_IF_ERROR(fh_transpose_batched(static_cast<int32_t>(x.dtype().itemsize()), x.raw_data(), y.raw_data(),
                                                 s.dim(0), s.dim(1), s.dim(2) * s.dim(3), stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

// channels_last of several tensors in one launch ([d0,d1,d2,d3] -> [d0,d2,d3,d1] each)
Status channels_last_multi_kernel(KernelContext& ctx) {
  const std::string op(kChannelsLastMultiOp);
  const size_t n = ctx.inputs.size();
  if (n == 0 || n > kMultiMaxTensors || ctx.outputs.size() != n) return invalid(op, "expects 1 to 32 inputs and as many outputs");
  std::vector<const void*> xs(n);
  std::vector<void*> ys(n);
  std::vector<int64_t> batch(n), rows(n), cols(n);
  const size_t itemsize = ctx.inputs[0].dtype().itemsize();
  for (size_t i = 0; i < n; ++i) {
    const Tensor& x = ctx.inputs[i];
    Tensor& y = ctx.outputs[i];
    const Shape& s = x.shape();
    if (s.rank() != 4 || !same_elem_type(x, y) || elem_bytes(x) != itemsize)
      return invalid(op, "expects rank-4 inputs of one item size, outputs of the same dtype");
    if (y.shape() != Shape({s.dim(0), s.dim(2), s.dim(3), s.dim(1)})) return invalid(op, "output shape does not match [d0,d2,d3,d1]");
    if (s.dim(1) * s.dim(2) * s.dim(3) > kMultiPlaneMax) return invalid(op, "planes above 8192 elements");
    xs[i] = x.raw_data();
    ys[i] = y.raw_data();
    batch[i] = s.dim(0);
    rows[i] = s.dim(1);
    cols[i] = s.dim(2) * s.dim(3);
  }
  FRAME_HIP_RETURN_IF_ERROR(fh_transpose_planes_multi(static_cast<int32_t>(itemsize), static_cast<int32_t>(n), xs.data(),
                                                      ys.data(), batch.data(), rows.data(), cols.data(),
                                                      stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

// x [N,C,H,W] (C <= 8) -> [N,H,W,8]
Status pack_input_c8_kernel(KernelContext& ctx) {
  const std::string op(kPackInputC8Op);
  FRAME_RETURN_IF_ERROR(arity(ctx, op, 1, 1));
  const Tensor& x = ctx.inputs[0];
  Tensor& y = ctx.outputs[0];
  const Shape& s = x.shape();
  if (s.rank() != 4 || elem_bytes(x) != 2 || y.shape() != Shape({s.dim(0), s.dim(2), s.dim(3), 8}))
    return invalid(op, "expects a 16-bit [N,C,H,W] input and a [N,H,W,8] output");
  FRAME_HIP_RETURN_IF_ERROR(fh_conv_pack_input_c8(x.raw_data(), y.raw_data(), s.dim(0), static_cast<int32_t>(s.dim(1)),
                                                  s.dim(2) * s.dim(3), stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

// w [Cout,C,KH,KW] (C <= 8) -> [Cout, K8]
Status pack_filter_c8_kernel(KernelContext& ctx) {
  const std::string op(kPackFilterC8Op);
  FRAME_RETURN_IF_ERROR(arity(ctx, op, 1, 1));
  const Tensor& w = ctx.inputs[0];
  Tensor& y = ctx.outputs[0];
  const Shape& s = w.shape();
  if (s.rank() != 4 || elem_bytes(w) != 2 || y.shape() != Shape({s.dim(0), fh_conv_c8_filter_k(s.dim(2), s.dim(3))}))
    return invalid(op, "expects a 16-bit [Cout,C,KH,KW] filter and a [Cout,K8] output");
  FRAME_HIP_RETURN_IF_ERROR(fh_conv_pack_filter_c8(w.raw_data(), y.raw_data(), static_cast<int32_t>(s.dim(0)),
                                                   static_cast<int32_t>(s.dim(1)), static_cast<int32_t>(s.dim(2)),
                                                   static_cast<int32_t>(s.dim(3)), stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

Status conv2d_kernel(KernelContext& ctx) {
  if (ctx.inputs.size() != 2 && ctx.inputs.size() != 3) return invalid("conv2d", "expects 2 or 3 inputs");
  return conv_impl(ctx, "conv2d", ctx.inputs.size());
}

Status conv_epilogue_kernel(KernelContext& ctx) {
  const auto* n_main = attr<int64_t>(ctx, "n_main_inputs");
  return conv_impl(ctx, std::string(kConvEpilogueOp), n_main ? static_cast<size_t>(*n_main) : 2);
}

// ---- row reductions ---------------------------------------------------------------------------------------

Status softmax_kernel(KernelContext& ctx) {
  FRAME_RETURN_IF_ERROR(arity(ctx, "softmax", 1, 1));
  FRAME_RETURN_IF_ERROR(same_dtype(ctx, "softmax"));
  const Tensor& x = ctx.inputs[0];
  if (x.shape().rank() != 2 || !(ctx.outputs[0].shape() == x.shape())) return invalid("softmax", "expects matching rank-2 tensors");
  Result<int32_t> dt = float_code("softmax", x.dtype());
  if (!dt.is_ok()) return dt.status();
  FRAME_HIP_RETURN_IF_ERROR(fh_softmax_rows(dt.value(), x.raw_data(), ctx.outputs[0].raw_data(), x.shape().dim(0),
                                            x.shape().dim(1), stream_handle(ctx)),
                            "op 'softmax' (hip)");
  return Status::ok();
}

// Fused attention produced by HipBackend::compile from the per-(batch, head) decomposition
// (reference: src/nn/layers.cpp:1014-1080); q, k, v, out are [batch*seq, heads*dh].
Status attention_kernel(KernelContext& ctx) {
  const std::string op(kAttentionOp);
  FRAME_RETURN_IF_ERROR(arity(ctx, op, 3, 1));
  FRAME_RETURN_IF_ERROR(same_dtype(ctx, op));
  const auto* batch = attr<int64_t>(ctx, "batch");
  const auto* seq = attr<int64_t>(ctx, "seq");
  const auto* heads = attr<int64_t>(ctx, "heads");
  const auto* dh = attr<int64_t>(ctx, "dh");
  const auto* scale = attr<double>(ctx, "scale");
  if (!batch || !seq || !heads || !dh || !scale) return invalid(op, "missing batch/seq/heads/dh/scale attributes");
  const Shape want({*batch * *seq, *heads * *dh});
  for (const Tensor& t : ctx.inputs)
    if (t.shape() != want) return invalid(op, "q, k, v must be [batch*seq, heads*dh]");
  if (ctx.outputs[0].shape() != want) return invalid(op, "out must be [batch*seq, heads*dh]");
  Result<int32_t> dt = float_code(op, ctx.outputs[0].dtype());
  if (!dt.is_ok()) return dt.status();
  FRAME_HIP_RETURN_IF_ERROR(fh_attention_fwd(dt.value(), ctx.inputs[0].raw_data(), ctx.inputs[1].raw_data(),
                                             ctx.inputs[2].raw_data(), ctx.outputs[0].raw_data(), *batch, *seq, *heads,
                                             *dh, static_cast<float>(*scale), stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

Status layer_norm_kernel(KernelContext& ctx) {
  FRAME_RETURN_IF_ERROR(arity(ctx, "layer_norm", 3, 1));
  FRAME_RETURN_IF_ERROR(same_dtype(ctx, "layer_norm"));
  const Tensor& x = ctx.inputs[0];
  const auto* eps = attr<double>(ctx, "eps");
  if (eps == nullptr) return invalid("layer_norm", "missing attribute 'eps'");
  if (x.shape().rank() != 2 || ctx.inputs[1].numel() != x.shape().dim(1) || ctx.inputs[2].numel() != x.shape().dim(1))
    return invalid("layer_norm", "expects x [N, D], gamma [D], beta [D]");
  Result<int32_t> dt = float_code("layer_norm", x.dtype());
  if (!dt.is_ok()) return dt.status();
  FRAME_HIP_RETURN_IF_ERROR(fh_layer_norm_rows(dt.value(), x.raw_data(), ctx.inputs[1].raw_data(), ctx.inputs[2].raw_data(),
                                               ctx.outputs[0].raw_data(), x.shape().dim(0), x.shape().dim(1),
                                               static_cast<float>(*eps), stream_handle(ctx)),
                            "op 'layer_norm' (hip)");
  return Status::ok();
}

template <int Mode>
Status pool_kernel(KernelContext& ctx) {
  const std::string op = Mode == 0 ? "max_pool2d" : "avg_pool2d";
  FRAME_RETURN_IF_ERROR(arity(ctx, op, 1, 1));
  FRAME_RETURN_IF_ERROR(same_dtype(ctx, op));
  const auto* k = attr<std::vector<int64_t>>(ctx, "kernel");
  const auto* s = attr<std::vector<int64_t>>(ctx, "stride");
  const auto* p = attr<std::vector<int64_t>>(ctx, "padding");
  if (!k || !s || !p || k->size() != 2 || s->size() != 2 || p->size() != 2) return invalid(op, "missing or malformed attributes");
  const Tensor& x = ctx.inputs[0];
  if (x.shape().rank() != 4) return invalid(op, "expects rank-4 input");
  Result<int32_t> dt = float_code(op, x.dtype());
  if (!dt.is_ok()) return dt.status();
  const int64_t geom[10] = {x.shape().dim(0), x.shape().dim(1), x.shape().dim(2), x.shape().dim(3), (*k)[0],
                            (*k)[1],          (*s)[0],          (*s)[1],          (*p)[0],          (*p)[1]};
  const int64_t oh = (geom[2] + 2 * geom[8] - geom[4]) / geom[6] + 1;
  const int64_t ow = (geom[3] + 2 * geom[9] - geom[5]) / geom[7] + 1;
  if (ctx.outputs[0].shape() != Shape({geom[0], geom[1], oh, ow})) return invalid(op, "output shape does not match the geometry");
  FRAME_HIP_RETURN_IF_ERROR(fh_pool2d(dt.value(), Mode, x.raw_data(), ctx.outputs[0].raw_data(), geom, stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

// ---- training path -----------------------------------------------------------------------------------------

// Geometry array of fh_pool2d / fh_pool2d_grad for input dims `x` and the op's kernel/stride/padding attributes.
Result<std::array<int64_t, 10>> pool_geom(KernelContext& ctx, const std::string& op, const Shape& x) {
  const auto* k = attr<std::vector<int64_t>>(ctx, "kernel");
  const auto* s = attr<std::vector<int64_t>>(ctx, "stride");
  const auto* p = attr<std::vector<int64_t>>(ctx, "padding");
  if (!k || !s || !p || k->size() != 2 || s->size() != 2 || p->size() != 2) return invalid(op, "missing or malformed attributes");
  if (x.rank() != 4) return invalid(op, "expects a rank-4 input_shape");
  return std::array<int64_t, 10>{x.dim(0), x.dim(1), x.dim(2), x.dim(3), (*k)[0], (*k)[1], (*s)[0], (*s)[1], (*p)[0], (*p)[1]};
}

// matmul_grad_lhs_internal (gy [m,n], b [k,n]) -> [m,k]; matmul_grad_rhs_internal (a [m,k], gy [m,n]) -> [k,n].
template <int Rhs>
Status matmul_grad_kernel(KernelContext& ctx) {
  const std::string op = Rhs ? "matmul_grad_rhs_internal" : "matmul_grad_lhs_internal";
  FRAME_RETURN_IF_ERROR(arity(ctx, op, 2, 1));
  FRAME_RETURN_IF_ERROR(same_dtype(ctx, op));
  const Shape& p = ctx.inputs[0].shape();
  const Shape& q = ctx.inputs[1].shape();
  if (p.rank() != 2 || q.rank() != 2) return invalid(op, "expects rank-2 operands");
  const int64_t m = p.dim(0), n = Rhs ? q.dim(1) : p.dim(1), k = Rhs ? p.dim(1) : q.dim(0);
  if ((Rhs ? q.dim(0) : q.dim(1)) != (Rhs ? m : n)) return invalid(op, "contraction dimension mismatch");
  if (ctx.outputs[0].shape() != (Rhs ? Shape({k, n}) : Shape({m, k}))) return invalid(op, "output shape mismatch");
  Result<int32_t> dt = float_code(op, ctx.outputs[0].dtype());
  if (!dt.is_ok()) return dt.status();
  FRAME_HIP_RETURN_IF_ERROR(fh_matmul_grad(dt.value(), Rhs, ctx.inputs[0].raw_data(), ctx.inputs[1].raw_data(),
                                           ctx.outputs[0].raw_data(), m, n, k, stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

template <int Mode>
Status pool_grad_kernel(KernelContext& ctx) {
  const std::string op = Mode == 0 ? "max_pool2d_grad_internal"
                         : Mode == 1 ? "avg_pool2d_grad_internal"
                                     : std::string(kMaxPoolReluGradOp);
  FRAME_RETURN_IF_ERROR(arity(ctx, op, Mode == 1 ? 1 : 2, 1));
  FRAME_RETURN_IF_ERROR(same_dtype(ctx, op));
  const Shape* xs = attr<Shape>(ctx, "input_shape");
  if (xs == nullptr) return invalid(op, "missing attribute 'input_shape'");
  Result<std::array<int64_t, 10>> g = pool_geom(ctx, op, *xs);
  if (!g.is_ok()) return g.status();
  if (ctx.outputs[0].shape() != *xs) return invalid(op, "output shape does not match input_shape");
  if (Mode != 1 && ctx.inputs[1].shape() != *xs) return invalid(op, "x shape does not match input_shape");
  const auto& geom = g.value();
  const int64_t oh = (geom[2] + 2 * geom[8] - geom[4]) / geom[6] + 1, ow = (geom[3] + 2 * geom[9] - geom[5]) / geom[7] + 1;
  if (ctx.inputs[0].shape() != Shape({geom[0], geom[1], oh, ow})) return invalid(op, "dy shape does not match the geometry");
  Result<int32_t> dt = float_code(op, ctx.outputs[0].dtype());
  if (!dt.is_ok()) return dt.status();
  FRAME_HIP_RETURN_IF_ERROR(fh_pool2d_grad(dt.value(), Mode, ctx.inputs[0].raw_data(),
                                           Mode != 1 ? ctx.inputs[1].raw_data() : nullptr, ctx.outputs[0].raw_data(),
                                           geom.data(), stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

// conv2d_grad_input_internal (dy, w) -> dx of input_shape; conv2d_grad_filter_internal (x, dy) -> dw of filter_shape.
template <int Filter>
Status conv_grad_kernel(KernelContext& ctx) {
  const std::string op = Filter ? "conv2d_grad_filter_internal" : "conv2d_grad_input_internal";
  FRAME_RETURN_IF_ERROR(arity(ctx, op, 2, 1));
  FRAME_RETURN_IF_ERROR(same_dtype(ctx, op));
  const Shape* fixed = attr<Shape>(ctx, Filter ? "filter_shape" : "input_shape");
  const auto* s = attr<std::vector<int64_t>>(ctx, "stride");
  const auto* p = attr<std::vector<int64_t>>(ctx, "padding");
  const auto* grp = attr<int64_t>(ctx, "groups");
  if (!fixed || !s || !p || !grp || s->size() != 2 || p->size() != 2) return invalid(op, "missing or malformed attributes");
  const Shape& x = Filter ? ctx.inputs[0].shape() : *fixed;
  const Shape& w = Filter ? *fixed : ctx.inputs[1].shape();
  if (x.rank() != 4 || w.rank() != 4) return invalid(op, "expects rank-4 x and w");
  if (ctx.outputs[0].shape() != *fixed) return invalid(op, "output shape does not match its shape attribute");
  const int64_t geom[12] = {x.dim(0), x.dim(1), x.dim(2), x.dim(3), w.dim(0), w.dim(2), w.dim(3), (*s)[0], (*s)[1], (*p)[0], (*p)[1], *grp};
  if (*grp <= 0 || (*s)[0] <= 0 || (*s)[1] <= 0) return invalid(op, "invalid stride or groups");
  const int64_t oh = (geom[2] + 2 * geom[9] - geom[5]) / geom[7] + 1, ow = (geom[3] + 2 * geom[10] - geom[6]) / geom[8] + 1;
  const Tensor& dy = ctx.inputs[Filter ? 1 : 0];
  if (dy.shape() != Shape({geom[0], geom[4], oh, ow}) || w.dim(1) * *grp != x.dim(1))
    return invalid(op, "dy / w shapes do not match the geometry");
  Result<int32_t> dt = float_code(op, ctx.outputs[0].dtype());
  if (!dt.is_ok()) return dt.status();
  if (Filter)
    FRAME_HIP_RETURN_IF_ERROR(fh_conv2d_grad_filter(dt.value(), ctx.inputs[0].raw_data(), dy.raw_data(), ctx.outputs[0].raw_data(),
                                                    geom, stream_handle(ctx)),
                              "op '" + op + "' (hip)");
  else
    FRAME_HIP_RETURN_IF_ERROR(fh_conv2d_grad_input(dt.value(), dy.raw_data(), ctx.inputs[1].raw_data(), ctx.outputs[0].raw_data(),
                                                   geom, stream_handle(ctx)),
                              "op '" + op + "' (hip)");
  return Status::ok();
}

// Sum over every axis but the last (kSumRowsOp); output 1 is the partials workspace.
Status sum_rows_kernel(KernelContext& ctx) {
  const std::string op(kSumRowsOp);
  if (ctx.inputs.size() != 1 || ctx.outputs.size() != 2) return invalid(op, "expects 1 input and 2 outputs");
  const Shape& x = ctx.inputs[0].shape();
  if (x.rank() < 1 || !same_elem_type(ctx.inputs[0], ctx.outputs[0])) return invalid(op, "operand shapes");
  const int64_t cols = x.dim(x.rank() - 1);
  if (ctx.outputs[0].numel() != cols) return invalid(op, "output must hold one value per column");
  Result<int32_t> dt = float_code(op, ctx.outputs[0].dtype());
  if (!dt.is_ok()) return dt.status();
  FRAME_HIP_RETURN_IF_ERROR(fh_sum_rows(dt.value(), ctx.inputs[0].raw_data(), ctx.outputs[0].raw_data(), x.numel() / cols, cols,
                                        ctx.outputs[1].raw_data(), ctx.outputs[1].numel() * 4, stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

// out_i = x_i + s_i * y_i over the pairs of kAxpyMultiOp (inputs [x_0, y_0, x_1, y_1, ...]), one launch.
Status axpy_multi_kernel(KernelContext& ctx) {
  const std::string op(kAxpyMultiOp);
  const size_t n = ctx.outputs.size();
  if (n == 0 || n > FH_AXPY_MAX || ctx.inputs.size() != 2 * n) return invalid(op, "expects 2 inputs per output, at most 32 outputs");
  const auto* scales = attr<std::vector<double>>(ctx, "scales");
  if (scales == nullptr || scales->size() != n) return invalid(op, "attribute 'scales' must hold one value per output");
  Result<int32_t> dt = float_code(op, ctx.outputs[0].dtype());
  if (!dt.is_ok()) return dt.status();
  const void* xs[FH_AXPY_MAX];
  const void* ys[FH_AXPY_MAX];
  void* outs[FH_AXPY_MAX];
  int64_t numel[FH_AXPY_MAX];
  float sv[FH_AXPY_MAX];
  for (size_t i = 0; i < n; ++i) {
    const Tensor& x = ctx.inputs[2 * i];
    const Tensor& y = ctx.inputs[2 * i + 1];
    Tensor& o = ctx.outputs[i];
    if (!same_elem_type(x, o) || !same_elem_type(y, o) || !same_elem_type(o, ctx.outputs[0]) ||
        x.shape() != o.shape() || y.shape() != o.shape())
      return invalid(op, "every pair must match its output's dtype and shape");
    xs[i] = x.raw_data(), ys[i] = y.raw_data(), outs[i] = o.raw_data();
    numel[i] = o.numel(), sv[i] = static_cast<float>((*scales)[i]);
  }
  FRAME_HIP_RETURN_IF_ERROR(fh_axpy_multi(dt.value(), static_cast<int32_t>(n), xs, ys, outs, numel, sv, stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

// avg_pool2d_grad_internal on channels-last dy [N,Ho,Wo,C] -> dx [N,H,W,C] (kAvgPoolGradNhwcOp).
Status avg_pool_grad_nhwc_kernel(KernelContext& ctx) {
  const std::string op(kAvgPoolGradNhwcOp);
  FRAME_RETURN_IF_ERROR(arity(ctx, op, 1, 1));
  FRAME_RETURN_IF_ERROR(same_dtype(ctx, op));
  const Shape* xs = attr<Shape>(ctx, "input_shape");  // NCHW input_shape of the forward
  if (xs == nullptr) return invalid(op, "missing attribute 'input_shape'");
  Result<std::array<int64_t, 10>> g = pool_geom(ctx, op, *xs);
  if (!g.is_ok()) return g.status();
  const auto& geom = g.value();
  const int64_t oh = (geom[2] + 2 * geom[8] - geom[4]) / geom[6] + 1, ow = (geom[3] + 2 * geom[9] - geom[5]) / geom[7] + 1;
  if (ctx.outputs[0].shape() != Shape({geom[0], geom[2], geom[3], geom[1]}) ||
      ctx.inputs[0].shape() != Shape({geom[0], oh, ow, geom[1]}))
    return invalid(op, "channels-last shapes do not match the geometry");
  Result<int32_t> dt = float_code(op, ctx.outputs[0].dtype());
  if (!dt.is_ok()) return dt.status();
  FRAME_HIP_RETURN_IF_ERROR(fh_avg_pool2d_grad_nhwc(dt.value(), ctx.inputs[0].raw_data(), ctx.outputs[0].raw_data(), geom.data(),
                                                    stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

// conv2d_grad_filter on MFMA over channels-last operands (kConvWgradOp); output 1 is the split-K workspace.
Status conv_wgrad_kernel(KernelContext& ctx) {
  const std::string op(kConvWgradOp);
  if (ctx.inputs.size() != 2 || ctx.outputs.size() != 2) return invalid(op, "expects 2 inputs and 2 outputs");
  const Shape* ws = attr<Shape>(ctx, "filter_shape");
  const auto* s = attr<std::vector<int64_t>>(ctx, "stride");
  const auto* p = attr<std::vector<int64_t>>(ctx, "padding");
  const auto* grp = attr<int64_t>(ctx, "groups");
  if (!ws || !s || !p || !grp || s->size() != 2 || p->size() != 2 || ws->rank() != 4) return invalid(op, "missing attributes");
  const Shape& x = ctx.inputs[0].shape();   // [N,H,W,cin_pad]
  const Shape& dy = ctx.inputs[1].shape();  // [N,Ho,Wo,Cout]
  if (x.rank() != 4 || dy.rank() != 4 || ctx.outputs[0].shape() != *ws) return invalid(op, "operand shapes");
  if (!same_elem_type(ctx.inputs[0], ctx.outputs[0]) || !same_elem_type(ctx.inputs[1], ctx.outputs[0]))
    return invalid(op, "operand dtypes differ");
  const int64_t geom[12] = {x.dim(0), ws->dim(1), x.dim(1), x.dim(2), ws->dim(0), ws->dim(2), ws->dim(3), (*s)[0], (*s)[1], (*p)[0], (*p)[1], *grp};
  const int64_t oh = (geom[2] + 2 * geom[9] - geom[5]) / geom[7] + 1, ow = (geom[3] + 2 * geom[10] - geom[6]) / geom[8] + 1;
  if (dy != Shape({geom[0], oh, ow, geom[4]}) || x.dim(3) < ws->dim(1)) return invalid(op, "dy / x shapes do not match the geometry");
  Result<int32_t> dt = float_code(op, ctx.outputs[0].dtype());
  if (!dt.is_ok()) return dt.status();
  const int64_t bytes = ctx.outputs[1].numel() * 4;
  FRAME_HIP_RETURN_IF_ERROR(fh_conv2d_wgrad_nhwc(dt.value(), ctx.inputs[0].raw_data(), ctx.inputs[1].raw_data(),
                                                 ctx.outputs[0].raw_data(), ctx.outputs[1].raw_data(), bytes, geom,
                                                 static_cast<int32_t>(x.dim(3)), stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

// Operands of the lowered conv2d_grad_input (see kFilterFlipOp / kDilateNhwcOp).
Status filter_flip_kernel(KernelContext& ctx) {
  const std::string op(kFilterFlipOp);
  FRAME_RETURN_IF_ERROR(arity(ctx, op, 1, 1));
  FRAME_RETURN_IF_ERROR(same_dtype(ctx, op));
  const Shape& w = ctx.inputs[0].shape();
  if (w.rank() != 4 || ctx.outputs[0].shape() != Shape({w.dim(1), w.dim(2), w.dim(3), w.dim(0)}))
    return invalid(op, "expects w [Cout,Cin,KH,KW] -> [Cin,KH,KW,Cout]");
  Result<int32_t> dt = float_code(op, ctx.outputs[0].dtype());
  if (!dt.is_ok()) return dt.status();
  FRAME_HIP_RETURN_IF_ERROR(fh_conv_filter_flip(dt.value(), ctx.inputs[0].raw_data(), ctx.outputs[0].raw_data(), w.dim(0),
                                                w.dim(1), w.dim(2), w.dim(3), stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

Status filter_flip_multi_kernel(KernelContext& ctx) {
  const std::string op(kFilterFlipMultiOp);
  const size_t n = ctx.inputs.size();
  if (n == 0 || n > FH_FLIP_MAX || ctx.outputs.size() != n) return invalid(op, "expects 1 to 32 inputs and as many outputs");
  Result<int32_t> dt = float_code(op, ctx.outputs[0].dtype());
  if (!dt.is_ok()) return dt.status();
  std::vector<const void*> ws(n);
  std::vector<void*> outs(n);
  std::vector<int64_t> dims(4 * n);
  for (size_t i = 0; i < n; ++i) {
    const Shape& w = ctx.inputs[i].shape();
    if (!same_elem_type(ctx.inputs[i], ctx.outputs[i]) || !same_elem_type(ctx.outputs[i], ctx.outputs[0]))
      return invalid(op, "expects inputs and outputs of one element type");
    if (w.rank() != 4 || ctx.outputs[i].shape() != Shape({w.dim(1), w.dim(2), w.dim(3), w.dim(0)}))
      return invalid(op, "expects w [Cout,Cin,KH,KW] -> [Cin,KH,KW,Cout]");
    ws[i] = ctx.inputs[i].raw_data();
    outs[i] = ctx.outputs[i].raw_data();
    for (int d = 0; d < 4; ++d) dims[4 * i + d] = w.dim(d);
  }
  FRAME_HIP_RETURN_IF_ERROR(fh_conv_filter_flip_multi(dt.value(), static_cast<int32_t>(n), ws.data(), outs.data(),
                                                      dims.data(), stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

Status dilate_nhwc_kernel(KernelContext& ctx) {
  const std::string op(kDilateNhwcOp);
  FRAME_RETURN_IF_ERROR(arity(ctx, op, 1, 1));
  FRAME_RETURN_IF_ERROR(same_dtype(ctx, op));
  const auto* s = attr<std::vector<int64_t>>(ctx, "stride");
  const Shape& x = ctx.inputs[0].shape();
  const Shape& y = ctx.outputs[0].shape();
  if (s == nullptr || s->size() != 2 || (*s)[0] < 1 || (*s)[1] < 1) return invalid(op, "missing or malformed stride");
  if (x.rank() != 4 || y.rank() != 4 || y.dim(0) != x.dim(0)) return invalid(op, "expects rank-4 tensors of one batch");
  Result<int32_t> dt = float_code(op, ctx.outputs[0].dtype());
  if (!dt.is_ok()) return dt.status();
  const auto* in_nhwc = attr<int64_t>(ctx, "in_nhwc");
  const bool cl = in_nhwc != nullptr && *in_nhwc != 0;
  // x NCHW [N,C,H,W], or channels-last [N,H,W,C]
  const int64_t xn = x.dim(0), xc = cl ? x.dim(3) : x.dim(1), xh = cl ? x.dim(1) : x.dim(2), xw = cl ? x.dim(2) : x.dim(3);
  if (y.dim(3) != xc || y.dim(1) < (xh - 1) * (*s)[0] + 1 || y.dim(2) < (xw - 1) * (*s)[1] + 1)
    return invalid(op, "output shape does not match the dilated input");
  FRAME_HIP_RETURN_IF_ERROR(fh_dilate_nhwc(dt.value(), cl ? 1 : 0, ctx.inputs[0].raw_data(), ctx.outputs[0].raw_data(), xn, xc,
                                           xh, xw, (*s)[0], (*s)[1], y.dim(1), y.dim(2), stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

// sum (x; axes[, keepdims]) and sum_grad_internal (gy; input_shape, axes): both index x's dims with a reduced mask.
template <int Grad>
Status sum_kernel(KernelContext& ctx) {
  const std::string op = Grad ? "sum_grad_internal" : "sum";
  FRAME_RETURN_IF_ERROR(arity(ctx, op, 1, 1));
  FRAME_RETURN_IF_ERROR(same_dtype(ctx, op));
  const auto* axes = attr<std::vector<int64_t>>(ctx, "axes");
  const Shape* xs_attr = Grad ? attr<Shape>(ctx, "input_shape") : nullptr;
  if (axes == nullptr || (Grad && xs_attr == nullptr)) return invalid(op, "missing attributes");
  const Shape& xs = Grad ? *xs_attr : ctx.inputs[0].shape();
  if (xs.rank() > 8) return Status::make(ErrorCode::kUnimplemented, "op '" + op + "' (hip): rank above 8");
  std::vector<uint8_t> red(static_cast<size_t>(xs.rank()), axes->empty() ? 1 : 0);
  for (int64_t a : *axes) {
    if (a < 0 || a >= xs.rank()) return invalid(op, "axis out of range");
    red[static_cast<size_t>(a)] = 1;
  }
  int64_t nout = 1;
  for (int64_t d = 0; d < xs.rank(); ++d)
    if (!red[static_cast<size_t>(d)]) nout *= xs.dim(d);
  if (Grad ? (ctx.outputs[0].shape() != xs || ctx.inputs[0].numel() != nout) : ctx.outputs[0].numel() != nout)
    return invalid(op, "input / output shapes do not match the axes");
  Result<int32_t> dt = float_code(op, ctx.outputs[0].dtype());
  if (!dt.is_ok()) return dt.status();
  if (Grad)
    FRAME_HIP_RETURN_IF_ERROR(fh_sum_grad(dt.value(), ctx.inputs[0].raw_data(), ctx.outputs[0].raw_data(),
                                          static_cast<int32_t>(xs.rank()), xs.dims().data(), red.data(), stream_handle(ctx)),
                              "op '" + op + "' (hip)");
  else
    FRAME_HIP_RETURN_IF_ERROR(fh_sum(dt.value(), ctx.inputs[0].raw_data(), ctx.outputs[0].raw_data(),
                                     static_cast<int32_t>(xs.rank()), xs.dims().data(), red.data(), stream_handle(ctx)),
                              "op '" + op + "' (hip)");
  return Status::ok();
}

template <int Grad>
Status mse_kernel(KernelContext& ctx) {
  const std::string op = Grad ? "mse_loss_grad_internal" : "mse_loss";
  FRAME_RETURN_IF_ERROR(arity(ctx, op, Grad ? 3 : 2, 1));
  FRAME_RETURN_IF_ERROR(same_dtype(ctx, op));
  const Tensor& p = ctx.inputs[0];
  if (ctx.inputs[1].shape() != p.shape()) return invalid(op, "pred and target shapes differ");
  if (Grad ? (ctx.outputs[0].shape() != p.shape() || ctx.inputs[2].numel() != 1) : ctx.outputs[0].numel() != 1)
    return invalid(op, "output / gy shapes do not match");
  Result<int32_t> dt = float_code(op, p.dtype());
  if (!dt.is_ok()) return dt.status();
  if (Grad)
    FRAME_HIP_RETURN_IF_ERROR(fh_mse_loss_grad(dt.value(), p.raw_data(), ctx.inputs[1].raw_data(), ctx.inputs[2].raw_data(),
                                               ctx.outputs[0].raw_data(), p.numel(), stream_handle(ctx)),
                              "op '" + op + "' (hip)");
  else
    FRAME_HIP_RETURN_IF_ERROR(fh_mse_loss(dt.value(), p.raw_data(), ctx.inputs[1].raw_data(), ctx.outputs[0].raw_data(),
                                          p.numel(), stream_handle(ctx)),
                              "op '" + op + "' (hip)");
  return Status::ok();
}

// Channels-last pooling on [N,H,W,C] activations (internal ops of the channels-last lowering), same attributes.
template <int Mode>
Status pool_nhwc_kernel(KernelContext& ctx) {
  const std::string op(Mode == 0 ? kMaxPoolNhwcOp : kAvgPoolNhwcOp);
  FRAME_RETURN_IF_ERROR(arity(ctx, op, 1, 1));
  FRAME_RETURN_IF_ERROR(same_dtype(ctx, op));
  const auto* k = attr<std::vector<int64_t>>(ctx, "kernel");
  const auto* s = attr<std::vector<int64_t>>(ctx, "stride");
  const auto* p = attr<std::vector<int64_t>>(ctx, "padding");
  if (!k || !s || !p || k->size() != 2 || s->size() != 2 || p->size() != 2) return invalid(op, "missing or malformed attributes");
  const Tensor& x = ctx.inputs[0];
  if (x.shape().rank() != 4) return invalid(op, "expects rank-4 input");
  Result<int32_t> dt = float_code(op, x.dtype());
  if (!dt.is_ok()) return dt.status();
  const int64_t geom[10] = {x.shape().dim(0), x.shape().dim(3), x.shape().dim(1), x.shape().dim(2), (*k)[0],
                            (*k)[1],          (*s)[0],          (*s)[1],          (*p)[0],          (*p)[1]};
  const int64_t oh = (geom[2] + 2 * geom[8] - geom[4]) / geom[6] + 1;
  const int64_t ow = (geom[3] + 2 * geom[9] - geom[5]) / geom[7] + 1;
  // a 1x1 output plane may come typed [N, C] (the same bytes; a reshape folded into the pool)
  const bool flat = oh == 1 && ow == 1 && ctx.outputs[0].shape() == Shape({geom[0], geom[1]});
  if (!flat && ctx.outputs[0].shape() != Shape({geom[0], oh, ow, geom[1]}))
    return invalid(op, "output shape does not match the geometry");
  FRAME_HIP_RETURN_IF_ERROR(fh_pool2d_nhwc(dt.value(), Mode, x.raw_data(), ctx.outputs[0].raw_data(), geom,
                                           stream_handle(ctx)),
                            "op '" + op + "' (hip)");
  return Status::ok();
}

// ---- data movement (bit-exact, any dtype) -----------------------------------------------------------------

Status reshape_kernel(KernelContext& ctx) {
  FRAME_RETURN_IF_ERROR(arity(ctx, "reshape", 1, 1));
  const Tensor& x = ctx.inputs[0];
  Tensor& y = ctx.outputs[0];
  if (x.numel() != y.numel() || !same_elem_type(x, y))
    return invalid("reshape", "element count or dtype differs");
  FRAME_HIP_RETURN_IF_ERROR(fh_memcpy(y.raw_data(), x.raw_data(), static_cast<size_t>(x.numel()) * x.dtype().itemsize(),
                                      FH_D2D, stream_handle(ctx)),
                            "op 'reshape' (hip)");
  return Status::ok();
}

Status transpose_kernel(KernelContext& ctx) {
  FRAME_RETURN_IF_ERROR(arity(ctx, "transpose", 1, 1));
  const Tensor& x = ctx.inputs[0];
  const auto* perm = attr<std::vector<int64_t>>(ctx, "perm");
  const int64_t r = x.shape().rank();
  if (perm == nullptr || static_cast<int64_t>(perm->size()) != r || r > 8) return invalid("transpose", "bad 'perm' or rank above 8");
  const auto& st = x.strides().values();
  std::vector<int64_t> out_dims, in_strides;
  for (int64_t d = 0; d < r; ++d) {
    const int64_t p = (*perm)[static_cast<size_t>(d)];
    if (p < 0 || p >= r) return invalid("transpose", "perm entry out of range");
    out_dims.push_back(x.shape().dim(p));
    in_strides.push_back(st[static_cast<size_t>(p)]);
  }
  if (ctx.outputs[0].shape() != Shape(out_dims)) return invalid("transpose", "output shape does not match perm");
  if (x.numel() == 0) return Status::ok();
  FRAME_HIP_RETURN_IF_ERROR(fh_permute(static_cast<int32_t>(x.dtype().itemsize()), x.raw_data(), ctx.outputs[0].raw_data(),
                                       static_cast<int32_t>(r), out_dims.data(), in_strides.data(), stream_handle(ctx)),
                            "op 'transpose' (hip)");
  return Status::ok();
}

// Row-major tensor seen as [outer, dim(axis) * inner] bytes around `axis`.
void split_at_axis(const Shape& s, int64_t axis, size_t item, int64_t& outer, int64_t& inner_bytes) {
  outer = 1;
  for (int64_t d = 0; d < axis; ++d) outer *= s.dim(d);
  int64_t inner = 1;
  for (int64_t d = axis + 1; d < s.rank(); ++d) inner *= s.dim(d);
  inner_bytes = inner * static_cast<int64_t>(item);
}

Status slice_kernel(KernelContext& ctx) {
  FRAME_RETURN_IF_ERROR(arity(ctx, "slice", 1, 1));
  const Tensor& x = ctx.inputs[0];
  const auto* axis = attr<int64_t>(ctx, "axis");
  const auto* start = attr<int64_t>(ctx, "start");
  const auto* stop = attr<int64_t>(ctx, "stop");
  if (!axis || !start || !stop || *axis < 0 || *axis >= x.shape().rank() || !(0 <= *start && *start < *stop && *stop <= x.shape().dim(*axis)))
    return invalid("slice", "bad axis/start/stop");
  int64_t outer = 0, inner = 0;
  split_at_axis(x.shape(), *axis, x.dtype().itemsize(), outer, inner);
  const int64_t src_pitch = x.shape().dim(*axis) * inner;
  const int64_t width = (*stop - *start) * inner;
  if (ctx.outputs[0].numel() * static_cast<int64_t>(elem_bytes(x)) != outer * width) return invalid("slice", "output size mismatch");
  FRAME_HIP_RETURN_IF_ERROR(fh_copy2d(ctx.outputs[0].raw_data(), width, static_cast<const char*>(x.raw_data()) + *start * inner,
                                      src_pitch, width, outer, stream_handle(ctx)),
                            "op 'slice' (hip)");
  return Status::ok();
}

Status concat_kernel(KernelContext& ctx) {
  if (ctx.inputs.empty() || ctx.outputs.size() != 1) return invalid("concat", "expects >= 1 input and 1 output");
  const auto* axis = attr<int64_t>(ctx, "axis");
  Tensor& y = ctx.outputs[0];
  if (axis == nullptr || *axis < 0 || *axis >= y.shape().rank()) return invalid("concat", "bad axis");
  int64_t outer = 0, inner = 0;
  split_at_axis(y.shape(), *axis, y.dtype().itemsize(), outer, inner);
  const int64_t dst_pitch = y.shape().dim(*axis) * inner;
  int64_t offset = 0;
  for (const Tensor& x : ctx.inputs) {
    if (!same_elem_type(x, y) || x.shape().rank() != y.shape().rank())
      return invalid("concat", "operand dtype/rank differs");
    const int64_t width = x.shape().dim(*axis) * inner;
    if (offset + width > dst_pitch) return invalid("concat", "operands exceed the output along the axis");
    if (width > 0 && outer > 0)
      FRAME_HIP_RETURN_IF_ERROR(fh_copy2d(static_cast<char*>(y.raw_data()) + offset, dst_pitch, x.raw_data(), width, width,
                                          outer, stream_handle(ctx)),
                                "op 'concat' (hip)");
    offset += width;
  }
  if (offset != dst_pitch) return invalid("concat", "operands do not fill the output");
  return Status::ok();
}

// Eager constant: host fill, then a synchronous upload. Compiled graphs materialise constants at compile time.
Status constant_kernel(KernelContext& ctx) {
  FRAME_RETURN_IF_ERROR(arity(ctx, "constant", 0, 1));
  if (ctx.attrs == nullptr) return invalid("constant", "requires attrs");
  Tensor& y = ctx.outputs[0];
  const size_t bytes = static_cast<size_t>(y.numel()) * y.dtype().itemsize();
  std::vector<unsigned char> host(std::max<size_t>(bytes, 1));
  struct HostAlloc final : hal::Allocator {
    void* p;
    explicit HostAlloc(void* q) : p(q) {}
    Result<void*> allocate(size_t, size_t) override { return p; }
    void deallocate(void*) override {}
  } ha(host.data());
  Result<Tensor> h = Tensor::empty(y.shape(), y.dtype(), cpu_device(), ha);
  if (!h.is_ok()) return h.status();
  FRAME_RETURN_IF_ERROR(ops::fill_tensor_from_constant_attrs(*ctx.attrs, h.value()));
  if (bytes > 0) FRAME_HIP_RETURN_IF_ERROR(fh_memcpy(y.raw_data(), host.data(), bytes, FH_H2D, nullptr), "op 'constant' (hip)");
  return Status::ok();
}

}  // namespace

FRAME_REGISTER_KERNEL("add", kHipBackendName, (&ew_kernel<FH_EW_ADD, 2>));
FRAME_REGISTER_KERNEL("mul", kHipBackendName, (&ew_kernel<FH_EW_MUL, 2>));
FRAME_REGISTER_KERNEL("relu", kHipBackendName, (&ew_kernel<FH_EW_RELU, 1>));
FRAME_REGISTER_KERNEL("square", kHipBackendName, (&ew_kernel<FH_EW_SQUARE, 1>));
FRAME_REGISTER_KERNEL("gelu", kHipBackendName, (&ew_kernel<FH_EW_GELU, 1>));
FRAME_REGISTER_KERNEL(ops::kFusedElementwiseOpName, kHipBackendName, &fused_kernel);
FRAME_REGISTER_KERNEL(kEwProgramOp, kHipBackendName, &ew_program_kernel);
FRAME_REGISTER_KERNEL("matmul", kHipBackendName, &matmul_kernel);
FRAME_REGISTER_KERNEL(kGemmEpilogueOp, kHipBackendName, &gemm_epilogue_kernel);
FRAME_REGISTER_KERNEL(kGemmGroupedOp, kHipBackendName, &gemm_grouped_kernel);
FRAME_REGISTER_KERNEL("conv2d", kHipBackendName, &conv2d_kernel);
FRAME_REGISTER_KERNEL(kConvEpilogueOp, kHipBackendName, &conv_epilogue_kernel);
FRAME_REGISTER_KERNEL(kConvNhwcOp, kHipBackendName, &conv_nhwc_kernel);
FRAME_REGISTER_KERNEL(kChannelsLastOp, kHipBackendName, &channels_last_kernel);
FRAME_REGISTER_KERNEL(kChannelsLastMultiOp, kHipBackendName, &channels_last_multi_kernel);
FRAME_REGISTER_KERNEL(kConvStemPoolOp, kHipBackendName, &conv_stem_pool_kernel);
FRAME_REGISTER_KERNEL(kPackInputC8Op, kHipBackendName, &pack_input_c8_kernel);
FRAME_REGISTER_KERNEL(kPackFilterC8Op, kHipBackendName, &pack_filter_c8_kernel);
FRAME_REGISTER_KERNEL("softmax", kHipBackendName, &softmax_kernel);
FRAME_REGISTER_KERNEL(kAttentionOp, kHipBackendName, &attention_kernel);
FRAME_REGISTER_KERNEL("layer_norm", kHipBackendName, &layer_norm_kernel);
FRAME_REGISTER_KERNEL("max_pool2d", kHipBackendName, &pool_kernel<0>);
FRAME_REGISTER_KERNEL("avg_pool2d", kHipBackendName, &pool_kernel<1>);
FRAME_REGISTER_KERNEL(kMaxPoolNhwcOp, kHipBackendName, &pool_nhwc_kernel<0>);
FRAME_REGISTER_KERNEL(kAvgPoolNhwcOp, kHipBackendName, &pool_nhwc_kernel<1>);
FRAME_REGISTER_KERNEL("reshape", kHipBackendName, &reshape_kernel);
FRAME_REGISTER_KERNEL("transpose", kHipBackendName, &transpose_kernel);
FRAME_REGISTER_KERNEL("slice", kHipBackendName, &slice_kernel);
FRAME_REGISTER_KERNEL("concat", kHipBackendName, &concat_kernel);
FRAME_REGISTER_KERNEL(ops::kConstantOpName, kHipBackendName, &constant_kernel);
FRAME_REGISTER_KERNEL("relu_grad_internal", kHipBackendName, (&ew_kernel<FH_EW_RELU_GRAD, 2>));
FRAME_REGISTER_KERNEL("gelu_grad_internal", kHipBackendName, (&ew_kernel<FH_EW_GELU_GRAD, 2>));
FRAME_REGISTER_KERNEL("sigmoid", kHipBackendName, (&ew_kernel<FH_EW_SIGMOID, 1>));
FRAME_REGISTER_KERNEL("tanh", kHipBackendName, (&ew_kernel<FH_EW_TANH, 1>));
FRAME_REGISTER_KERNEL("rsqrt", kHipBackendName, (&ew_kernel<FH_EW_RSQRT, 1>));
FRAME_REGISTER_KERNEL("matmul_grad_lhs_internal", kHipBackendName, &matmul_grad_kernel<0>);
FRAME_REGISTER_KERNEL("matmul_grad_rhs_internal", kHipBackendName, &matmul_grad_kernel<1>);
FRAME_REGISTER_KERNEL("max_pool2d_grad_internal", kHipBackendName, &pool_grad_kernel<0>);
FRAME_REGISTER_KERNEL("avg_pool2d_grad_internal", kHipBackendName, &pool_grad_kernel<1>);
FRAME_REGISTER_KERNEL(kMaxPoolReluGradOp, kHipBackendName, &pool_grad_kernel<2>);
FRAME_REGISTER_KERNEL("conv2d_grad_input_internal", kHipBackendName, &conv_grad_kernel<0>);
FRAME_REGISTER_KERNEL("conv2d_grad_filter_internal", kHipBackendName, &conv_grad_kernel<1>);
FRAME_REGISTER_KERNEL(kFilterFlipOp, kHipBackendName, &filter_flip_kernel);
FRAME_REGISTER_KERNEL(kFilterFlipMultiOp, kHipBackendName, &filter_flip_multi_kernel);
FRAME_REGISTER_KERNEL(kConvWgradOp, kHipBackendName, &conv_wgrad_kernel);
FRAME_REGISTER_KERNEL(kAvgPoolGradNhwcOp, kHipBackendName, &avg_pool_grad_nhwc_kernel);
FRAME_REGISTER_KERNEL(kSumRowsOp, kHipBackendName, &sum_rows_kernel);
FRAME_REGISTER_KERNEL(kAxpyMultiOp, kHipBackendName, &axpy_multi_kernel);
FRAME_REGISTER_KERNEL(kDilateNhwcOp, kHipBackendName, &dilate_nhwc_kernel);
FRAME_REGISTER_KERNEL("sum", kHipBackendName, &sum_kernel<0>);
FRAME_REGISTER_KERNEL("sum_grad_internal", kHipBackendName, &sum_kernel<1>);
FRAME_REGISTER_KERNEL("mse_loss", kHipBackendName, &mse_kernel<0>);
FRAME_REGISTER_KERNEL("mse_loss_grad_internal", kHipBackendName, &mse_kernel<1>);

}  // namespace frame::backends::hip

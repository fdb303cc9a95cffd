// Op contracts of the compiled-graph forward path. Shape rules follow the reference schemas:
//   elementwise  src/ops/schemas/elementwise.cpp:41-62, 667-748 (no broadcasting; add/mul commutative)
//   matmul       src/ops/schemas/matmul.cpp:24-63, 281-286 (rank-2 only)
//   conv2d       src/ops/schemas/conv.cpp:60-200, 979-989 (NCHW, optional [Cout] bias, floor output size)
//   softmax / layer_norm  src/ops/schemas/sequence.cpp:335-347, 417-470, 635-649 (rank-2, last axis)
//   pooling      src/ops/schemas/pool.cpp:60-190, 596-614 (padding <= kernel/2)
//   shape ops    src/ops/schemas/shape.cpp:416-449
//   constant     src/ops/schemas/constant.cpp:127-132
//   fused chain  src/ops/schemas/fused_elementwise.cpp:24-51
// gelu has no counterpart in the reference: it is this build's addition (0.5*x*(1+erf(x/sqrt(2)))), declared
// elementwise and fusable so operator_fusion can merge bias-add + gelu into one fused group.
#include <cstdint>
#include <numeric>
#include <string>
#include <vector>

#include <frame/core/shape.h>
#include <frame/core/status.h>
#include <frame/ops/constant_utils.h>
#include <frame/ops/fused_elementwise_utils.h>
#include <frame/ops/op_registry.h>

#include "gradients.h"

namespace {

using frame::DType;
using frame::ErrorCode;
using frame::Result;
using frame::Shape;
using frame::Status;
using frame::ops::NodeContext;
using frame::ops::OpTrait;
using Shapes = Result<std::vector<Shape>>;
using frame::ir::AttrType;

Status bad(const std::string& op, const std::string& msg) {
  return Status::make(ErrorCode::kInvalidArgument, "op '" + op + "' " + msg);
}

std::string op_of(const NodeContext& c) { return std::string(c.op); }

Status expect_inputs(const NodeContext& c, size_t n) {
  if (c.input_types.size() != n)
    return bad(op_of(c), "expects " + std::to_string(n) + " input" + (n == 1 ? "" : "s") + ", got " +
                             std::to_string(c.input_types.size()));
  return Status::ok();
}

int64_t floor_div(int64_t a, int64_t b) { return a >= 0 ? a / b : -((-a + b - 1) / b); }

Shapes unary_same(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect_inputs(c, 1));
  return std::vector<Shape>{c.input_types[0].shape};
}

Shapes binary_same(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect_inputs(c, 2));
  const auto& a = c.input_types[0];
  const auto& b = c.input_types[1];
  if (!(a.dtype == b.dtype))
    return bad(op_of(c), "requires lhs and rhs of the same dtype, got '" + std::string(a.dtype.name()) + "' and '" +
                             std::string(b.dtype.name()) + "'");
  if (!(a.shape == b.shape))
    return bad(op_of(c), "requires lhs and rhs of the same shape (v0 has no broadcasting), got " +
                             a.shape.to_string() + " and " + b.shape.to_string());
  return std::vector<Shape>{a.shape};
}

Shapes infer_matmul(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect_inputs(c, 2));
  const auto& a = c.input_types[0];
  const auto& b = c.input_types[1];
  if (a.shape.rank() != 2) return bad("matmul", "requires lhs to be rank-2, got rank " + std::to_string(a.shape.rank()));
  if (b.shape.rank() != 2) return bad("matmul", "requires rhs to be rank-2, got rank " + std::to_string(b.shape.rank()));
  if (!(a.dtype == b.dtype))
    return bad("matmul", "requires lhs and rhs of the same dtype, got '" + std::string(a.dtype.name()) + "' and '" +
                             std::string(b.dtype.name()) + "'");
  if (a.shape.dim(1) != b.shape.dim(0))
    return bad("matmul", "contraction dimension mismatch: lhs " + a.shape.to_string() + " has k=" +
                             std::to_string(a.shape.dim(1)) + ", rhs " + b.shape.to_string() + " has k=" +
                             std::to_string(b.shape.dim(0)) +
                             " (lhs's last dimension must equal rhs's first dimension)");
  return std::vector<Shape>{Shape({a.shape.dim(0), b.shape.dim(1)})};
}

Result<std::vector<int64_t>> pair_attr(const NodeContext& c, const char* name) {
  const auto* v = c.attr<std::vector<int64_t>>(name);
  if (v == nullptr) return bad(op_of(c), std::string("is missing required attribute '") + name + "' (int64 array)");
  if (v->size() != 2)
    return bad(op_of(c), std::string("attribute '") + name + "' must have 2 entries, got " + std::to_string(v->size()));
  return *v;
}

Shapes infer_conv2d(const NodeContext& c) {
  const std::string op = "conv2d";
  if (c.input_types.size() < 2)
    return bad(op, "expects at least 2 inputs (x, w), got " + std::to_string(c.input_types.size()));
  if (c.input_types.size() > 3)
    return bad(op, "bias group expects at most 1 tensor, got " + std::to_string(c.input_types.size() - 2));
  const auto& x = c.input_types[0];
  const auto& w = c.input_types[1];
  if (!(x.dtype == w.dtype))
    return bad(op, "requires x and w of the same dtype, got '" + std::string(x.dtype.name()) + "' and '" +
                       std::string(w.dtype.name()) + "'");
  Result<std::vector<int64_t>> stride = pair_attr(c, "stride");
  if (!stride.is_ok()) return stride.status();
  Result<std::vector<int64_t>> pad = pair_attr(c, "padding");
  if (!pad.is_ok()) return pad.status();
  const int64_t* groups = c.attr<int64_t>("groups");
  if (groups == nullptr) return bad(op, "is missing required attribute 'groups'");
  if (x.shape.rank() != 4) return bad(op, "requires x to be rank-4 [N, Cin, H, W], got rank " + std::to_string(x.shape.rank()));
  if (w.shape.rank() != 4)
    return bad(op, "requires w to be rank-4 [Cout, Cin/groups, KH, KW], got rank " + std::to_string(w.shape.rank()));
  if (*groups < 1) return bad(op, "attribute 'groups' must be >= 1, got " + std::to_string(*groups));
  const int64_t n = x.shape.dim(0), cin = x.shape.dim(1), h = x.shape.dim(2), wd = x.shape.dim(3);
  const int64_t cout = w.shape.dim(0), cpg = w.shape.dim(1), kh = w.shape.dim(2), kw = w.shape.dim(3);
  const auto& s = stride.value();
  const auto& p = pad.value();
  if (n <= 0 || cin <= 0 || h <= 0 || wd <= 0) return bad(op, "requires x dims to be positive, got " + x.shape.to_string());
  if (cout <= 0 || cpg <= 0 || kh <= 0 || kw <= 0) return bad(op, "requires w dims to be positive, got " + w.shape.to_string());
  if (s[0] < 1 || s[1] < 1) return bad(op, "attribute 'stride' entries must be >= 1");
  if (p[0] < 0 || p[1] < 0) return bad(op, "attribute 'padding' entries must be >= 0");
  if (cin % *groups != 0) return bad(op, "Cin=" + std::to_string(cin) + " is not divisible by groups=" + std::to_string(*groups));
  if (cout % *groups != 0) return bad(op, "Cout=" + std::to_string(cout) + " is not divisible by groups=" + std::to_string(*groups));
  if (cpg != cin / *groups)
    return bad(op, "w's second dimension (Cin/groups) is " + std::to_string(cpg) + ", expected " + std::to_string(cin / *groups));
  const int64_t oh = floor_div(h + 2 * p[0] - kh, s[0]) + 1;
  const int64_t ow = floor_div(wd + 2 * p[1] - kw, s[1]) + 1;
  if (oh < 1) return bad(op, "produces non-positive output height " + std::to_string(oh));
  if (ow < 1) return bad(op, "produces non-positive output width " + std::to_string(ow));
  if (c.input_types.size() == 3) {
    const auto& b = c.input_types[2];
    if (!(b.dtype == x.dtype)) return bad(op, "requires bias and x of the same dtype");
    if (b.shape.rank() != 1) return bad(op, "requires bias to be rank-1, got rank " + std::to_string(b.shape.rank()));
    if (b.shape.dim(0) != cout)
      return bad(op, "requires bias size to equal Cout=" + std::to_string(cout) + ", got " + std::to_string(b.shape.dim(0)));
  }
  return std::vector<Shape>{Shape({n, cout, oh, ow})};
}

Shapes infer_pool(const NodeContext& c) {
  const std::string op = op_of(c);
  FRAME_RETURN_IF_ERROR(expect_inputs(c, 1));
  Result<std::vector<int64_t>> k = pair_attr(c, "kernel");
  if (!k.is_ok()) return k.status();
  Result<std::vector<int64_t>> s = pair_attr(c, "stride");
  if (!s.is_ok()) return s.status();
  Result<std::vector<int64_t>> p = pair_attr(c, "padding");
  if (!p.is_ok()) return p.status();
  const Shape& x = c.input_types[0].shape;
  if (x.rank() != 4) return bad(op, "requires x to be rank-4 [N, C, H, W], got rank " + std::to_string(x.rank()));
  if (x.dim(0) <= 0 || x.dim(1) <= 0 || x.dim(2) <= 0 || x.dim(3) <= 0)
    return bad(op, "requires x dims [N, C, H, W] to be positive, got " + x.to_string());
  const auto &kk = k.value(), &ss = s.value(), &pp = p.value();
  if (kk[0] < 1 || kk[1] < 1) return bad(op, "attribute 'kernel' entries must be >= 1");
  if (ss[0] < 1 || ss[1] < 1) return bad(op, "attribute 'stride' entries must be >= 1");
  if (pp[0] < 0 || pp[1] < 0) return bad(op, "attribute 'padding' entries must be >= 0");
  if (pp[0] * 2 > kk[0]) return bad(op, "padding_h*2=" + std::to_string(pp[0] * 2) + " exceeds KH=" + std::to_string(kk[0]));
  if (pp[1] * 2 > kk[1]) return bad(op, "padding_w*2=" + std::to_string(pp[1] * 2) + " exceeds KW=" + std::to_string(kk[1]));
  const int64_t oh = floor_div(x.dim(2) + 2 * pp[0] - kk[0], ss[0]) + 1;
  const int64_t ow = floor_div(x.dim(3) + 2 * pp[1] - kk[1], ss[1]) + 1;
  if (oh < 1) return bad(op, "produces non-positive output height " + std::to_string(oh));
  if (ow < 1) return bad(op, "produces non-positive output width " + std::to_string(ow));
  return std::vector<Shape>{Shape({x.dim(0), x.dim(1), oh, ow})};
}

Shapes infer_softmax(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect_inputs(c, 1));
  const Shape& x = c.input_types[0].shape;
  if (x.rank() != 2) return bad("softmax", "requires x to be rank-2 [N, D], got rank " + std::to_string(x.rank()));
  return std::vector<Shape>{x};
}

Shapes infer_layer_norm(const NodeContext& c) {
  const std::string op = "layer_norm";
  FRAME_RETURN_IF_ERROR(expect_inputs(c, 3));
  const auto& x = c.input_types[0];
  if (x.shape.rank() != 2) return bad(op, "requires x to be rank-2 [N, D], got rank " + std::to_string(x.shape.rank()));
  const int64_t d = x.shape.dim(1);
  for (size_t i = 1; i < 3; ++i) {
    const auto& t = c.input_types[i];
    const std::string nm = i == 1 ? "gamma" : "beta";
    if (t.shape.rank() != 1) return bad(op, "requires " + nm + " to be rank-1, got rank " + std::to_string(t.shape.rank()));
    if (t.shape.dim(0) != d) return bad(op, "requires " + nm + " size to equal D=" + std::to_string(d));
    if (!(t.dtype == x.dtype)) return bad(op, "requires " + nm + " and x of the same dtype");
  }
  if (c.attr<double>("eps") == nullptr) return bad(op, "is missing required attribute 'eps' (double)");
  return std::vector<Shape>{x.shape};
}

Shapes infer_reshape(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect_inputs(c, 1));
  const Shape* t = c.attr<Shape>("target_shape");
  if (t == nullptr) return bad("reshape", "is missing required attribute 'target_shape' (shape)");
  FRAME_RETURN_IF_ERROR(t->verify());
  if (t->numel() != c.input_types[0].shape.numel())
    return bad("reshape", "target_shape " + t->to_string() + " has " + std::to_string(t->numel()) +
                              " element(s), input " + c.input_types[0].shape.to_string() + " has " +
                              std::to_string(c.input_types[0].shape.numel()));
  return std::vector<Shape>{*t};
}

Shapes infer_transpose(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect_inputs(c, 1));
  const auto* perm = c.attr<std::vector<int64_t>>("perm");
  if (perm == nullptr) return bad("transpose", "is missing required attribute 'perm' (int64 array)");
  const Shape& x = c.input_types[0].shape;
  if (static_cast<int64_t>(perm->size()) != x.rank())
    return bad("transpose", "attribute 'perm' has " + std::to_string(perm->size()) + " entries, input rank is " +
                                std::to_string(x.rank()));
  std::vector<bool> seen(perm->size(), false);
  std::vector<int64_t> dims;
  for (int64_t p : *perm) {
    if (p < 0 || p >= x.rank() || seen[static_cast<size_t>(p)])
      return bad("transpose", "attribute 'perm' is not a permutation of [0, rank)");
    seen[static_cast<size_t>(p)] = true;
    dims.push_back(x.dim(p));
  }
  return std::vector<Shape>{Shape(dims)};
}

Shapes infer_slice(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect_inputs(c, 1));
  const int64_t* axis = c.attr<int64_t>("axis");
  const int64_t* start = c.attr<int64_t>("start");
  const int64_t* stop = c.attr<int64_t>("stop");
  if (axis == nullptr || start == nullptr || stop == nullptr)
    return bad("slice", "is missing one of the required attributes 'axis', 'start', 'stop'");
  const Shape& x = c.input_types[0].shape;
  if (*axis < 0 || *axis >= x.rank()) return bad("slice", "axis " + std::to_string(*axis) + " is out of range for rank " + std::to_string(x.rank()));
  if (!(0 <= *start && *start < *stop && *stop <= x.dim(*axis)))
    return bad("slice", "requires 0 <= start < stop <= dim, got start=" + std::to_string(*start) + ", stop=" +
                            std::to_string(*stop) + ", dim=" + std::to_string(x.dim(*axis)));
  std::vector<int64_t> dims = x.dims();
  dims[static_cast<size_t>(*axis)] = *stop - *start;
  return std::vector<Shape>{Shape(dims)};
}

Shapes infer_concat(const NodeContext& c) {
  if (c.input_types.empty()) return bad("concat", "expects at least 1 input, got 0");
  const int64_t* axis = c.attr<int64_t>("axis");
  if (axis == nullptr) return bad("concat", "is missing required attribute 'axis'");
  const auto& x0 = c.input_types[0];
  if (*axis < 0 || *axis >= x0.shape.rank())
    return bad("concat", "axis " + std::to_string(*axis) + " is out of range for rank " + std::to_string(x0.shape.rank()));
  std::vector<int64_t> dims = x0.shape.dims();
  for (size_t i = 1; i < c.input_types.size(); ++i) {
    const auto& t = c.input_types[i];
    if (!(t.dtype == x0.dtype)) return bad("concat", "requires all inputs to share a dtype");
    if (t.shape.rank() != x0.shape.rank()) return bad("concat", "requires all inputs to share a rank");
    for (int64_t d = 0; d < t.shape.rank(); ++d)
      if (d != *axis && t.shape.dim(d) != x0.shape.dim(d))
        return bad("concat", "input " + std::to_string(i) + " shape " + t.shape.to_string() +
                                 " differs from input 0 shape " + x0.shape.to_string() + " outside the axis");
    dims[static_cast<size_t>(*axis)] += t.shape.dim(*axis);
  }
  return std::vector<Shape>{Shape(dims)};
}

Shapes infer_constant(const NodeContext& c) {
  if (!c.input_types.empty()) return bad("constant", "expects 0 inputs, got " + std::to_string(c.input_types.size()));
  const Shape* s = c.attr<Shape>("shape");
  if (s == nullptr) return bad("constant", "is missing required attribute 'shape'");
  const auto* v = c.attr<std::vector<double>>("value");
  if (v != nullptr && static_cast<int64_t>(v->size()) != s->numel())
    return bad("constant", "attribute 'value' has " + std::to_string(v->size()) + " element(s), attribute 'shape' " +
                               s->to_string() + " expects " + std::to_string(s->numel()));
  return std::vector<Shape>{*s};
}

Shapes infer_fused(const NodeContext& c) {
  if (c.input_types.empty()) return bad("fused_elementwise_internal", "expects at least 1 input, got 0");
  if (c.attrs == nullptr) return bad("fused_elementwise_internal", "requires non-null attrs");
  frame::ops::FusedElementwiseChain chain;
  FRAME_RETURN_IF_ERROR(
      frame::ops::decode_and_validate_fused_chain(*c.attrs, static_cast<int64_t>(c.input_types.size()), chain));
  return std::vector<Shape>{c.input_types[0].shape};
}

}  // namespace

FRAME_REGISTER_OP("add")
    .input("lhs", "left operand")
    .input("rhs", "right operand")
    .output("out", "elementwise sum")
    .trait(OpTrait::kElementwise)
    .trait(OpTrait::kFusable)
    .trait(OpTrait::kCommutative)
    .shape_infer(&binary_same)
    .gradient(&frame::ops::schemas::add_gradient);

FRAME_REGISTER_OP("mul")
    .input("lhs", "left operand")
    .input("rhs", "right operand")
    .output("out", "elementwise product")
    .trait(OpTrait::kElementwise)
    .trait(OpTrait::kFusable)
    .trait(OpTrait::kCommutative)
    .shape_infer(&binary_same)
    .gradient(&frame::ops::schemas::mul_gradient);

FRAME_REGISTER_OP("relu")
    .input("x", "input")
    .output("out", "max(x, 0), NaN kept")
    .trait(OpTrait::kElementwise)
    .trait(OpTrait::kFusable)
    .shape_infer(&unary_same)
    .gradient(&frame::ops::schemas::relu_gradient);

FRAME_REGISTER_OP("square")
    .input("x", "input")
    .output("out", "x * x")
    .trait(OpTrait::kElementwise)
    .trait(OpTrait::kFusable)
    .shape_infer(&unary_same)
    .gradient(&frame::ops::schemas::square_gradient);

FRAME_REGISTER_OP("gelu")
    .input("x", "input")
    .output("out", "0.5 * x * (1 + erf(x / sqrt(2)))")
    .trait(OpTrait::kElementwise)
    .trait(OpTrait::kFusable)
    .shape_infer(&unary_same)
    .gradient(&frame::ops::schemas::gelu_gradient);

FRAME_REGISTER_OP("sigmoid").input("x", "input").output("out", "1 / (1 + exp(-x))").trait(OpTrait::kElementwise).shape_infer(&unary_same)
    .gradient(&frame::ops::schemas::sigmoid_gradient);
FRAME_REGISTER_OP("tanh").input("x", "input").output("out", "tanh(x)").trait(OpTrait::kElementwise).shape_infer(&unary_same)
    .gradient(&frame::ops::schemas::tanh_gradient);
FRAME_REGISTER_OP("rsqrt").input("x", "input").output("out", "1 / sqrt(x)").trait(OpTrait::kElementwise).shape_infer(&unary_same)
    .gradient(&frame::ops::schemas::rsqrt_gradient);

FRAME_REGISTER_OP("matmul")
    .input("lhs", "rank-2 [m, k]")
    .input("rhs", "rank-2 [k, n]")
    .output("out", "rank-2 [m, n]")
    .shape_infer(&infer_matmul)
    .gradient(&frame::ops::schemas::matmul_gradient);

FRAME_REGISTER_OP("conv2d")
    .input("x", "rank-4 [N, Cin, H, W]")
    .input("w", "rank-4 [Cout, Cin/groups, KH, KW]")
    .variadic_input("bias", "optional rank-1 [Cout]", 0)
    .attr("stride", AttrType::kInt64Array, true)
    .attr("padding", AttrType::kInt64Array, true)
    .attr("groups", AttrType::kInt64, true)
    .output("out", "rank-4 [N, Cout, out_h, out_w]")
    .shape_infer(&infer_conv2d)
    .gradient(&frame::ops::schemas::conv2d_gradient);

FRAME_REGISTER_OP("softmax").input("x", "rank-2 [N, D]").output("out", "softmax along the last axis").shape_infer(&infer_softmax)
    .gradient(&frame::ops::schemas::softmax_gradient);

FRAME_REGISTER_OP("layer_norm")
    .input("x", "rank-2 [N, D]")
    .input("gamma", "rank-1 [D]")
    .input("beta", "rank-1 [D]")
    .attr("eps", AttrType::kDouble, true)
    .output("out", "row-wise layer normalisation with affine")
    .shape_infer(&infer_layer_norm)
    .gradient(&frame::ops::schemas::layer_norm_gradient);

FRAME_REGISTER_OP("max_pool2d")
    .input("x", "rank-4 [N, C, H, W]")
    .attr("kernel", AttrType::kInt64Array, true)
    .attr("stride", AttrType::kInt64Array, true)
    .attr("padding", AttrType::kInt64Array, true)
    .output("out", "max pooling; padding is -inf")
    .shape_infer(&infer_pool)
    .gradient(&frame::ops::schemas::max_pool2d_gradient);

FRAME_REGISTER_OP("avg_pool2d")
    .input("x", "rank-4 [N, C, H, W]")
    .attr("kernel", AttrType::kInt64Array, true)
    .attr("stride", AttrType::kInt64Array, true)
    .attr("padding", AttrType::kInt64Array, true)
    .output("out", "average pooling; denominator KH*KW")
    .shape_infer(&infer_pool)
    .gradient(&frame::ops::schemas::avg_pool2d_gradient);

FRAME_REGISTER_OP("reshape").input("x", "input").attr("target_shape", AttrType::kShape, true).output("out", "reshaped x").shape_infer(&infer_reshape)
    .gradient(&frame::ops::schemas::reshape_gradient);
FRAME_REGISTER_OP("transpose").input("x", "input").attr("perm", AttrType::kInt64Array, true).output("out", "out.dims[i] = x.dims[perm[i]]").shape_infer(&infer_transpose)
    .gradient(&frame::ops::schemas::transpose_gradient);
FRAME_REGISTER_OP("concat").variadic_input("xs", "tensors to concatenate", 1).attr("axis", AttrType::kInt64, true).output("out", "concatenation").shape_infer(&infer_concat)
    .gradient(&frame::ops::schemas::concat_gradient);
FRAME_REGISTER_OP("slice")
    .input("x", "input")
    .attr("axis", AttrType::kInt64, true)
    .attr("start", AttrType::kInt64, true)
    .attr("stop", AttrType::kInt64, true)
    .output("out", "x[start:stop] along axis")
    .shape_infer(&infer_slice)
    .gradient(&frame::ops::schemas::slice_gradient);

FRAME_REGISTER_OP(frame::ops::kConstantOpName)
    .attr("value", AttrType::kDoubleArray, true)
    .attr("shape", AttrType::kShape, true)
    .attr("dtype", AttrType::kDType, true)
    .output("out", "materialised constant")
    .shape_infer(&infer_constant);

FRAME_REGISTER_OP(frame::ops::kFusedElementwiseOpName)
    .variadic_input("inputs", "external inputs of the fused chain", 1)
    .output("out", "output of the fused chain")
    .attr("ops", AttrType::kString, true)
    .attr("arities", AttrType::kInt64Array, true)
    .trait(OpTrait::kElementwise)
    .shape_infer(&infer_fused);

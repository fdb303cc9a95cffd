// Gradient micrographs and the gradient-only ops of the training path. Node structure and order follow the
// reference so that compiler::build_backward_graph produces the same training graph:
//   add/mul/square/relu gradients   src/ops/schemas/elementwise.cpp:211-360, relu_grad_internal :753-758
//   matmul gradient + grad ops      src/ops/schemas/matmul.cpp:60-200, 281-303
//   conv2d gradient + grad ops      src/ops/schemas/conv.cpp:257-470, 995-1015
//   pool gradients + grad ops       src/ops/schemas/pool.cpp:230-420, 596-655
//   sum / sum_grad_internal         src/ops/schemas/reduction.cpp:30-301
//   mse_loss / mse_loss_grad        src/ops/schemas/loss.cpp:30-279
//   reshape / transpose / slice / concat gradients   src/ops/schemas/shape.cpp:60-410
//   softmax / layer_norm gradients and their row-statistics helpers   src/ops/schemas/sequence.cpp:255-615
//   sigmoid / tanh / rsqrt gradients   src/ops/schemas/elementwise.cpp:401-660
// gelu and gelu_grad_internal are this build's own (the reference has no gelu).
// Only first-order gradients are registered: the gradient-only ops carry no GradientFn here, so differentiating
// a training graph a second time reports kUnimplemented naming the op.
#include "gradients.h"

#include <string>
#include <vector>

#include <frame/core/shape.h>
#include <frame/core/status.h>
#include <frame/ops/constant_utils.h>
#include <frame/ops/graph_builder.h>
#include <frame/ops/op_registry.h>

namespace frame::ops::schemas {

namespace {

using Shapes = Result<std::vector<Shape>>;
using ir::AttrType;

Status bad(const std::string& op, const std::string& msg) {
  return Status::make(ErrorCode::kInvalidArgument, "op '" + op + "' " + msg);
}

// Shape inference of a registered op, run on a node context of our own making.
Shapes infer_as(std::string_view op, std::vector<ir::TensorType> inputs, const AttrMap* attrs) {
  const OpSchema* s = OpRegistry::instance().find(op);
  if (s == nullptr || s->shape_infer() == nullptr)
    return Status::make(ErrorCode::kInternal, "op '" + std::string(op) + "' has no shape inference");
  NodeContext c;
  c.op = op;
  c.input_types = std::move(inputs);
  c.attrs = attrs;
  return s->shape_infer()(c);
}

ir::TensorType with_shape(ir::TensorType t, const Shape& s) {
  t.shape = s;
  return t;
}

// Micrograph under construction: the first failure is kept and later calls become no-ops.
class Micro {
 public:
  explicit Micro(const char* name) : g_(name) {}
  ir::Value* in(const ir::TensorType& t) {
    if (!st_.is_ok()) return nullptr;
    Result<ir::Value*> v = g_.add_graph_input(t);
    if (!v.is_ok()) st_ = v.status();
    return v.is_ok() ? v.value() : nullptr;
  }
  ir::Value* op(std::string_view name, std::vector<ir::Value*> ins, const AttrMap& attrs = {}) {
    if (!st_.is_ok()) return nullptr;
    Result<ir::Node*> n = create_node_with_inferred_types(g_, name, std::move(ins), attrs);
    if (!n.is_ok()) st_ = n.status();
    return n.is_ok() ? n.value()->output(0) : nullptr;
  }
  ir::Value* splat_shape(const ir::TensorType& like, const Shape& shape, double v) {
    ir::TensorType t = like;
    t.shape = shape;
    return splat(t, v);
  }
  ir::Value* splat(const ir::TensorType& like, double v) {
    if (!st_.is_ok()) return nullptr;
    const AttrMap attrs{{"value", std::vector<double>(static_cast<size_t>(like.shape.numel()), v)},
                        {"shape", like.shape},
                        {"dtype", like.dtype}};
    Result<ir::Node*> n = create_node_with_inferred_types(g_, kConstantOpName, like.device, attrs);
    if (!n.is_ok()) st_ = n.status();
    return n.is_ok() ? n.value()->output(0) : nullptr;
  }
  void fail(Status s) {
    if (st_.is_ok()) st_ = std::move(s);
  }
  Result<ir::Graph> finish(const std::vector<ir::Value*>& outs) {
    for (ir::Value* v : outs)
      if (st_.is_ok()) st_ = g_.mark_output(v);
    if (!st_.is_ok()) return st_;
    return std::move(g_);
  }

 private:
  ir::Graph g_;
  Status st_ = Status::ok();
};

// Inputs [x.., y, gy] of a single-output forward op; y's type is the forward's inferred output.
struct Fwd {
  std::vector<ir::Value*> x;
  ir::Value* y = nullptr;
  ir::Value* gy = nullptr;
};

Fwd forward_inputs(Micro& m, const NodeContext& c) {
  Fwd f;
  for (const auto& t : c.input_types) f.x.push_back(m.in(t));
  Shapes ys = infer_as(c.op, c.input_types, c.attrs);
  if (!ys.is_ok()) {
    m.fail(ys.status());
    return f;
  }
  const ir::TensorType yt = with_shape(c.input_types[0], ys.value()[0]);
  f.y = m.in(yt);
  f.gy = m.in(yt);
  return f;
}

Status expect(const NodeContext& c, size_t n, const char* what) {
  if (c.input_types.size() != n)
    return bad(std::string(c.op), std::string("gradient expects ") + what + ", got " + std::to_string(c.input_types.size()));
  return Status::ok();
}

AttrMap pick(const NodeContext& c, std::initializer_list<const char*> names) {
  AttrMap out;
  if (c.attrs == nullptr) return out;
  for (const char* n : names)
    if (auto it = c.attrs->find(n); it != c.attrs->end()) out.emplace(n, it->second);
  return out;
}

// ---- shape inference of the gradient-only ops ------------------------------------------------------------

Status same_dtype(const std::string& op, const ir::TensorType& a, const ir::TensorType& b, const char* an, const char* bn) {
  if (!(a.dtype == b.dtype))
    return bad(op, std::string("requires ") + an + " and " + bn + " of the same dtype, got '" + std::string(a.dtype.name()) +
                       "' and '" + std::string(b.dtype.name()) + "'");
  return Status::ok();
}

Shapes infer_relu_grad(const NodeContext& c) {
  const std::string op = "relu_grad_internal";
  if (c.input_types.size() != 2) return bad(op, "expects 2 inputs, got " + std::to_string(c.input_types.size()));
  const auto &x = c.input_types[0], &gy = c.input_types[1];
  FRAME_RETURN_IF_ERROR(same_dtype(op, x, gy, "x", "gy"));
  if (!(x.shape == gy.shape))
    return bad(op, "requires x and gy of the same shape, got " + x.shape.to_string() + " and " + gy.shape.to_string());
  return std::vector<Shape>{x.shape};
}

Shapes infer_matmul_grad(const NodeContext& c, bool lhs) {
  const std::string op = lhs ? "matmul_grad_lhs_internal" : "matmul_grad_rhs_internal";
  if (c.input_types.size() != 2) return bad(op, "expects 2 inputs, got " + std::to_string(c.input_types.size()));
  const auto &p = c.input_types[0], &q = c.input_types[1];
  const char* pn = lhs ? "gy" : "a";
  const char* qn = lhs ? "b" : "gy";
  if (p.shape.rank() != 2) return bad(op, std::string("requires ") + pn + " to be rank-2, got rank " + std::to_string(p.shape.rank()));
  if (q.shape.rank() != 2) return bad(op, std::string("requires ") + qn + " to be rank-2, got rank " + std::to_string(q.shape.rank()));
  FRAME_RETURN_IF_ERROR(same_dtype(op, p, q, pn, qn));
  if (lhs) {  // gy [m,n], b [k,n] -> [m,k]
    if (p.shape.dim(1) != q.shape.dim(1))
      return bad(op, "contraction dimension mismatch: gy " + p.shape.to_string() + " has n=" + std::to_string(p.shape.dim(1)) +
                         ", b " + q.shape.to_string() + " has n=" + std::to_string(q.shape.dim(1)));
    return std::vector<Shape>{Shape({p.shape.dim(0), q.shape.dim(0)})};
  }
  // a [m,k], gy [m,n] -> [k,n]
  if (p.shape.dim(0) != q.shape.dim(0))
    return bad(op, "contraction dimension mismatch: a " + p.shape.to_string() + " has m=" + std::to_string(p.shape.dim(0)) +
                       ", gy " + q.shape.to_string() + " has m=" + std::to_string(q.shape.dim(0)));
  return std::vector<Shape>{Shape({p.shape.dim(1), q.shape.dim(1)})};
}
Shapes infer_matmul_grad_lhs(const NodeContext& c) { return infer_matmul_grad(c, true); }
Shapes infer_matmul_grad_rhs(const NodeContext& c) { return infer_matmul_grad(c, false); }

Result<Shape> static_shape_attr(const NodeContext& c, const std::string& op, const char* name) {
  const Shape* s = c.attr<Shape>(name);
  if (s == nullptr) return bad(op, std::string("is missing required attribute '") + name + "'");
  if (s->has_dynamic_dim())
    return bad(op, std::string("attribute '") + name + "' " + s->to_string() + " has a dynamic dimension, static shape required");
  return *s;
}

Shapes infer_conv_grad_input(const NodeContext& c) {
  const std::string op = "conv2d_grad_input_internal";
  if (c.input_types.size() != 2) return bad(op, "expects 2 inputs, got " + std::to_string(c.input_types.size()));
  const auto &dy = c.input_types[0], &w = c.input_types[1];
  FRAME_RETURN_IF_ERROR(same_dtype(op, dy, w, "dy", "w"));
  Result<Shape> xs = static_shape_attr(c, op, "input_shape");
  if (!xs.is_ok()) return xs.status();
  Shapes y = infer_as("conv2d", {with_shape(dy, xs.value()), w}, c.attrs);
  if (!y.is_ok()) return bad(op, std::string(y.status().message()));
  if (!(y.value()[0] == dy.shape))
    return bad(op, "requires dy shape to be consistent with input_shape/w/stride/padding/groups, got " + dy.shape.to_string() +
                       ", expected " + y.value()[0].to_string());
  return std::vector<Shape>{xs.value()};
}

Shapes infer_conv_grad_filter(const NodeContext& c) {
  const std::string op = "conv2d_grad_filter_internal";
  if (c.input_types.size() != 2) return bad(op, "expects 2 inputs, got " + std::to_string(c.input_types.size()));
  const auto &x = c.input_types[0], &dy = c.input_types[1];
  FRAME_RETURN_IF_ERROR(same_dtype(op, x, dy, "x", "dy"));
  Result<Shape> ws = static_shape_attr(c, op, "filter_shape");
  if (!ws.is_ok()) return ws.status();
  Shapes y = infer_as("conv2d", {x, with_shape(x, ws.value())}, c.attrs);
  if (!y.is_ok()) return bad(op, std::string(y.status().message()));
  if (!(y.value()[0] == dy.shape))
    return bad(op, "requires dy shape to be consistent with x/filter_shape/stride/padding/groups, got " + dy.shape.to_string() +
                       ", expected " + y.value()[0].to_string());
  return std::vector<Shape>{ws.value()};
}

// dy must have the pooled shape of input_shape; max additionally takes x of shape input_shape.
Shapes infer_pool_grad(const NodeContext& c, bool is_max) {
  const std::string op = is_max ? "max_pool2d_grad_internal" : "avg_pool2d_grad_internal";
  const size_t n = is_max ? 2 : 1;
  if (c.input_types.size() != n) return bad(op, "expects " + std::to_string(n) + " input(s), got " + std::to_string(c.input_types.size()));
  const auto& dy = c.input_types[0];
  Result<Shape> xs = static_shape_attr(c, op, "input_shape");
  if (!xs.is_ok()) return xs.status();
  if (is_max) {
    const auto& x = c.input_types[1];
    FRAME_RETURN_IF_ERROR(same_dtype(op, dy, x, "dy", "x"));
    if (!(x.shape == xs.value()))
      return bad(op, "requires x shape to equal input_shape, got " + x.shape.to_string() + " and " + xs.value().to_string());
  }
  Shapes y = infer_as(is_max ? "max_pool2d" : "avg_pool2d", {with_shape(dy, xs.value())}, c.attrs);
  if (!y.is_ok()) return bad(op, std::string(y.status().message()));
  if (!(y.value()[0] == dy.shape))
    return bad(op, "requires dy shape to be consistent with input_shape/kernel/stride/padding, got " + dy.shape.to_string() +
                       ", expected " + y.value()[0].to_string());
  return std::vector<Shape>{xs.value()};
}
Shapes infer_max_pool_grad(const NodeContext& c) { return infer_pool_grad(c, true); }
Shapes infer_avg_pool_grad(const NodeContext& c) { return infer_pool_grad(c, false); }

// axes: empty = every axis; otherwise distinct, 0 <= axis < rank (no negative normalisation).
Status reduced_axes(const std::string& op, int64_t rank, const std::vector<int64_t>& axes, std::vector<bool>& reduced) {
  reduced.assign(static_cast<size_t>(rank), axes.empty());
  for (int64_t a : axes) {
    if (a < 0)
      return bad(op, "axes entry " + std::to_string(a) + " is negative; v0 requires 0 <= axis < rank and does not normalize negative indices");
    if (a >= rank)
      return bad(op, "axes entry " + std::to_string(a) + " is out of range for rank " + std::to_string(rank) + " (must satisfy 0 <= axis < rank)");
    if (reduced[static_cast<size_t>(a)]) return bad(op, "axes entry " + std::to_string(a) + " is duplicated");
    reduced[static_cast<size_t>(a)] = true;
  }
  return Status::ok();
}

Shape reduce_shape(const Shape& x, const std::vector<bool>& reduced, bool keepdims) {
  std::vector<int64_t> d;
  for (int64_t i = 0; i < x.rank(); ++i) {
    if (!reduced[static_cast<size_t>(i)]) d.push_back(x.dim(i));
    else if (keepdims) d.push_back(1);
  }
  return Shape(d);
}

Shapes infer_sum(const NodeContext& c) {
  if (c.input_types.size() != 1) return bad("sum", "expects 1 input, got " + std::to_string(c.input_types.size()));
  const auto* axes = c.attr<std::vector<int64_t>>("axes");
  if (axes == nullptr) return bad("sum", "is missing required attribute 'axes' (int64 array)");
  const bool* kd = c.attr<bool>("keepdims");
  std::vector<bool> red;
  FRAME_RETURN_IF_ERROR(reduced_axes("sum", c.input_types[0].shape.rank(), *axes, red));
  return std::vector<Shape>{reduce_shape(c.input_types[0].shape, red, kd != nullptr && *kd)};
}

// gy must be sum(input_shape, axes) with keepdims false or true; returns whether it is the keepdims form.
Result<bool> sum_grad_keepdims(const ir::TensorType& gy, const Shape& xs, const std::vector<int64_t>& axes) {
  std::vector<bool> red;
  FRAME_RETURN_IF_ERROR(reduced_axes("sum_grad_internal", xs.rank(), axes, red));
  const Shape squeezed = reduce_shape(xs, red, false), kept = reduce_shape(xs, red, true);
  const bool sq = gy.shape == squeezed, kp = gy.shape == kept;
  if (!sq && !kp)
    return bad("sum_grad_internal", "requires gy shape to match sum(input_shape, axes) with keepdims=false or true, got " +
                                        gy.shape.to_string() + ", expected " + squeezed.to_string() + " or " + kept.to_string());
  return kp && !sq;
}

Shapes infer_sum_grad(const NodeContext& c) {
  const std::string op = "sum_grad_internal";
  if (c.input_types.size() != 1) return bad(op, "expects 1 input, got " + std::to_string(c.input_types.size()));
  Result<Shape> xs = static_shape_attr(c, op, "input_shape");
  if (!xs.is_ok()) return xs.status();
  const auto* axes = c.attr<std::vector<int64_t>>("axes");
  if (axes == nullptr) return bad(op, "is missing required attribute 'axes' (int64 array)");
  Result<bool> kd = sum_grad_keepdims(c.input_types[0], xs.value(), *axes);
  if (!kd.is_ok()) return kd.status();
  return std::vector<Shape>{xs.value()};
}

Shapes infer_mse_loss(const NodeContext& c) {
  if (c.input_types.size() != 2) return bad("mse_loss", "expects 2 inputs, got " + std::to_string(c.input_types.size()));
  const auto &p = c.input_types[0], &t = c.input_types[1];
  FRAME_RETURN_IF_ERROR(same_dtype("mse_loss", p, t, "pred", "target"));
  if (!(p.shape == t.shape))
    return bad("mse_loss", "requires pred and target of the same shape, got " + p.shape.to_string() + " and " + t.shape.to_string());
  return std::vector<Shape>{Shape()};
}

Shapes infer_mse_loss_grad(const NodeContext& c) {
  const std::string op = "mse_loss_grad_internal";
  if (c.input_types.size() != 3) return bad(op, "expects 3 inputs, got " + std::to_string(c.input_types.size()));
  const auto &p = c.input_types[0], &t = c.input_types[1], &gy = c.input_types[2];
  FRAME_RETURN_IF_ERROR(same_dtype(op, p, t, "pred", "target"));
  if (!(p.shape == t.shape))
    return bad(op, "requires pred and target of the same shape, got " + p.shape.to_string() + " and " + t.shape.to_string());
  if (gy.shape.rank() != 0 && gy.shape.numel() != 1)
    return bad(op, "requires gy to be scalar (rank 0 or numel==1), got " + gy.shape.to_string());
  FRAME_RETURN_IF_ERROR(same_dtype(op, gy, p, "gy", "pred"));
  return std::vector<Shape>{p.shape};
}

// ---- first-order gradients of the gradient-path forward ops ------------------------------------------------

Result<ir::Graph> sum_gradient(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect(c, 1, "1 input"));
  const auto* axes = c.attr<std::vector<int64_t>>("axes");
  if (axes == nullptr)
    return bad("sum", "gradient is missing required attribute 'axes' (int64 array) on the original sum node");
  Micro m("sum_gradient");
  Fwd f = forward_inputs(m, c);
  ir::Value* gx = m.op("sum_grad_internal", {f.gy}, {{"input_shape", c.input_types[0].shape}, {"axes", *axes}});
  return m.finish({gx});
}

Result<ir::Graph> mse_loss_gradient(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect(c, 2, "2 inputs"));
  Micro m("mse_loss_gradient");
  Fwd f = forward_inputs(m, c);
  ir::Value* gpred = m.op("mse_loss_grad_internal", {f.x[0], f.x[1], f.gy});
  ir::Value* neg = m.splat(c.input_types[0], -1.0);
  ir::Value* gtarget = m.op("mul", {neg, gpred});
  return m.finish({gpred, gtarget});
}

// Row-statistics helpers of the softmax / layer_norm gradients (reference: src/ops/schemas/sequence.cpp:255-330):
// mean over axis 1 = sum * splat(1/d); a per-row [n] vector broadcast to [n,d] = reshape [n,1] @ ones [1,d]; a
// per-column [d] vector broadcast = ones [n,1] @ reshape [1,d]; a - b = a + (-1) * b.
ir::Value* mean_axis1(Micro& m, ir::Value* x, const ir::TensorType& t, int64_t n, int64_t d) {
  ir::Value* s = m.op("sum", {x}, {{"axes", std::vector<int64_t>{1}}});
  ir::Value* r = m.splat_shape(t, Shape({n}), 1.0 / static_cast<double>(d));
  return m.op("mul", {s, r});
}
ir::Value* bcast_col(Micro& m, ir::Value* v, const ir::TensorType& t, int64_t n, int64_t d) {
  ir::Value* col = m.op("reshape", {v}, {{"target_shape", Shape({n, 1})}});
  ir::Value* ones = m.splat_shape(t, Shape({1, d}), 1.0);
  return m.op("matmul", {col, ones});
}
ir::Value* bcast_row(Micro& m, ir::Value* v, const ir::TensorType& t, int64_t n, int64_t d) {
  ir::Value* row = m.op("reshape", {v}, {{"target_shape", Shape({1, d})}});
  ir::Value* ones = m.splat_shape(t, Shape({n, 1}), 1.0);
  return m.op("matmul", {ones, row});
}
ir::Value* minus(Micro& m, ir::Value* a, ir::Value* b, const ir::TensorType& t) {
  ir::Value* neg = m.splat(t, -1.0);
  return m.op("add", {a, m.op("mul", {neg, b})});
}

}  // namespace

Result<ir::Graph> add_gradient(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect(c, 2, "2 inputs"));
  Micro m("add_gradient");
  Fwd f = forward_inputs(m, c);
  return m.finish({f.gy, f.gy});
}

Result<ir::Graph> mul_gradient(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect(c, 2, "2 inputs"));
  Micro m("mul_gradient");
  Fwd f = forward_inputs(m, c);
  ir::Value* ga = m.op("mul", {f.gy, f.x[1]});
  ir::Value* gb = m.op("mul", {f.gy, f.x[0]});
  return m.finish({ga, gb});
}

Result<ir::Graph> relu_gradient(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect(c, 1, "1 input"));
  Micro m("relu_gradient");
  Fwd f = forward_inputs(m, c);
  return m.finish({m.op("relu_grad_internal", {f.x[0], f.gy})});
}

Result<ir::Graph> square_gradient(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect(c, 1, "1 input"));
  Micro m("square_gradient");
  Fwd f = forward_inputs(m, c);
  ir::Value* two = m.splat(c.input_types[0], 2.0);
  ir::Value* two_x = m.op("mul", {two, f.x[0]});
  return m.finish({m.op("mul", {f.gy, two_x})});
}

Result<ir::Graph> matmul_gradient(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect(c, 2, "2 inputs"));
  Micro m("matmul_gradient");
  Fwd f = forward_inputs(m, c);
  ir::Value* ga = m.op("matmul_grad_lhs_internal", {f.gy, f.x[1]});
  ir::Value* gb = m.op("matmul_grad_rhs_internal", {f.x[0], f.gy});
  return m.finish({ga, gb});
}

Result<ir::Graph> conv2d_gradient(const NodeContext& c) {
  if (c.input_types.size() < 2)
    return bad("conv2d", "gradient expects at least 2 inputs (x, w), got " + std::to_string(c.input_types.size()));
  if (c.input_types.size() > 3)
    return bad("conv2d", "gradient bias group expects at most 1 tensor, got " + std::to_string(c.input_types.size() - 2));
  Micro m("conv2d_gradient");
  Fwd f = forward_inputs(m, c);
  AttrMap gx_attrs = pick(c, {"stride", "padding", "groups"});
  gx_attrs.emplace("input_shape", c.input_types[0].shape);
  AttrMap gw_attrs = pick(c, {"stride", "padding", "groups"});
  gw_attrs.emplace("filter_shape", c.input_types[1].shape);
  ir::Value* gx = m.op("conv2d_grad_input_internal", {f.gy, f.x[1]}, gx_attrs);
  ir::Value* gw = m.op("conv2d_grad_filter_internal", {f.x[0], f.gy}, gw_attrs);
  std::vector<ir::Value*> outs{gx, gw};
  if (c.input_types.size() == 3) outs.push_back(m.op("sum", {f.gy}, {{"axes", std::vector<int64_t>{0, 2, 3}}}));
  return m.finish(outs);
}

namespace {
Result<ir::Graph> pool_gradient(const NodeContext& c, bool is_max) {
  FRAME_RETURN_IF_ERROR(expect(c, 1, "1 input"));
  Micro m(is_max ? "max_pool2d_gradient" : "avg_pool2d_gradient");
  Fwd f = forward_inputs(m, c);
  AttrMap a = pick(c, {"kernel", "stride", "padding"});
  a.emplace("input_shape", c.input_types[0].shape);
  ir::Value* gx = is_max ? m.op("max_pool2d_grad_internal", {f.gy, f.x[0]}, a) : m.op("avg_pool2d_grad_internal", {f.gy}, a);
  return m.finish({gx});
}
}  // namespace

Result<ir::Graph> max_pool2d_gradient(const NodeContext& c) { return pool_gradient(c, true); }
Result<ir::Graph> avg_pool2d_gradient(const NodeContext& c) { return pool_gradient(c, false); }

Result<ir::Graph> reshape_gradient(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect(c, 1, "1 input"));
  Micro m("reshape_gradient");
  Fwd f = forward_inputs(m, c);
  return m.finish({m.op("reshape", {f.gy}, {{"target_shape", c.input_types[0].shape}})});
}

// softmax (reference: src/ops/schemas/sequence.cpp:358-406): t = softmax(x) recomputed,
// gx = t * (gy - bcast_col(sum(t * gy, axis 1))).
Result<ir::Graph> softmax_gradient(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect(c, 1, "1 input"));
  Micro m("softmax_gradient");
  Fwd f = forward_inputs(m, c);
  const ir::TensorType& t = c.input_types[0];
  const int64_t n = t.shape.dim(0), d = t.shape.dim(1);
  ir::Value* sm = m.op("softmax", {f.x[0]});
  ir::Value* tg = m.op("mul", {sm, f.gy});
  ir::Value* s = m.op("sum", {tg}, {{"axes", std::vector<int64_t>{1}}});
  ir::Value* sb = bcast_col(m, s, t, n, d);
  ir::Value* diff = minus(m, f.gy, sb, t);
  return m.finish({m.op("mul", {sm, diff})});
}

// layer_norm (reference: src/ops/schemas/sequence.cpp:479-615): mean / variance / rsqrt recomputed from x, then
// gx = r * ((a - mean(a)) - xhat * mean(a * xhat)) with a = gamma * gy; ggamma = sum(gy * xhat, axis 0);
// gbeta = sum(gy, axis 0).
Result<ir::Graph> layer_norm_gradient(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect(c, 3, "3 inputs (x, gamma, beta)"));
  const auto* eps = c.attr<double>("eps");
  if (eps == nullptr) return bad("layer_norm", "gradient is missing attribute 'eps'");
  Micro m("layer_norm_gradient");
  Fwd f = forward_inputs(m, c);
  const ir::TensorType& t = c.input_types[0];
  const int64_t n = t.shape.dim(0), d = t.shape.dim(1);
  ir::Value* mu = mean_axis1(m, f.x[0], t, n, d);
  ir::Value* mub = bcast_col(m, mu, t, n, d);
  ir::Value* cen = minus(m, f.x[0], mub, t);
  ir::Value* sq = m.op("mul", {cen, cen});
  ir::Value* var = mean_axis1(m, sq, t, n, d);
  ir::Value* epsv = m.splat_shape(t, Shape({n}), *eps);
  ir::Value* ve = m.op("add", {var, epsv});
  ir::Value* r = m.op("rsqrt", {ve});
  ir::Value* rb = bcast_col(m, r, t, n, d);
  ir::Value* xhat = m.op("mul", {cen, rb});
  ir::Value* gb = bcast_row(m, f.x[1], t, n, d);
  ir::Value* a = m.op("mul", {gb, f.gy});
  ir::Value* ma = mean_axis1(m, a, t, n, d);
  ir::Value* mab = bcast_col(m, ma, t, n, d);
  ir::Value* ax = m.op("mul", {a, xhat});
  ir::Value* max = mean_axis1(m, ax, t, n, d);
  ir::Value* maxb = bcast_col(m, max, t, n, d);
  ir::Value* term1 = minus(m, a, mab, t);
  ir::Value* xm = m.op("mul", {xhat, maxb});
  ir::Value* term = minus(m, term1, xm, t);
  ir::Value* gx = m.op("mul", {rb, term});
  ir::Value* gyx = m.op("mul", {f.gy, xhat});
  ir::Value* gg = m.op("sum", {gyx}, {{"axes", std::vector<int64_t>{0}}});
  ir::Value* gbeta = m.op("sum", {f.gy}, {{"axes", std::vector<int64_t>{0}}});
  return m.finish({gx, gg, gbeta});
}

// transpose (reference: src/ops/schemas/shape.cpp:150-185): transpose of gy by the inverse permutation.
Result<ir::Graph> transpose_gradient(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect(c, 1, "1 input"));
  const auto* perm = c.attr<std::vector<int64_t>>("perm");
  if (perm == nullptr) return bad("transpose", "gradient is missing attribute 'perm'");
  std::vector<int64_t> inv(perm->size());
  for (size_t i = 0; i < perm->size(); ++i) inv[static_cast<size_t>((*perm)[i])] = static_cast<int64_t>(i);
  Micro m("transpose_gradient");
  Fwd f = forward_inputs(m, c);
  return m.finish({m.op("transpose", {f.gy}, {{"perm", inv}})});
}

// concat (reference: src/ops/schemas/shape.cpp:240-290): each input's gradient is its slice of gy along the axis.
Result<ir::Graph> concat_gradient(const NodeContext& c) {
  if (c.input_types.empty()) return bad("concat", "gradient expects at least 1 input, got 0");
  const auto* axis = c.attr<int64_t>("axis");
  if (axis == nullptr) return bad("concat", "gradient is missing attribute 'axis'");
  Micro m("concat_gradient");
  Fwd f = forward_inputs(m, c);
  std::vector<ir::Value*> outs;
  int64_t start = 0;
  for (const auto& t : c.input_types) {
    const int64_t stop = start + t.shape.dim(*axis);
    outs.push_back(m.op("slice", {f.gy}, {{"axis", *axis}, {"start", start}, {"stop", stop}}));
    start = stop;
  }
  return m.finish(outs);
}

// slice (reference: src/ops/schemas/shape.cpp:352-410): gy concatenated between zero blocks of the cut-off parts.
Result<ir::Graph> slice_gradient(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect(c, 1, "1 input"));
  const auto* axis = c.attr<int64_t>("axis");
  const auto* start = c.attr<int64_t>("start");
  const auto* stop = c.attr<int64_t>("stop");
  if (axis == nullptr || start == nullptr || stop == nullptr) return bad("slice", "gradient is missing attributes");
  Micro m("slice_gradient");
  Fwd f = forward_inputs(m, c);
  const ir::TensorType& t = c.input_types[0];
  const int64_t dim = t.shape.dim(*axis);
  std::vector<ir::Value*> parts;
  if (*start > 0) {
    std::vector<int64_t> dims = t.shape.dims();
    dims[static_cast<size_t>(*axis)] = *start;
    parts.push_back(m.splat_shape(t, Shape(dims), 0.0));
  }
  parts.push_back(f.gy);
  if (*stop < dim) {
    std::vector<int64_t> dims = t.shape.dims();
    dims[static_cast<size_t>(*axis)] = dim - *stop;
    parts.push_back(m.splat_shape(t, Shape(dims), 0.0));
  }
  return m.finish({m.op("concat", parts, {{"axis", *axis}})});
}

// sigmoid (reference: src/ops/schemas/elementwise.cpp:401-470): s = sigmoid(x) recomputed, gx = gy * (s * (1 - s)).
Result<ir::Graph> sigmoid_gradient(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect(c, 1, "1 input"));
  Micro m("sigmoid_gradient");
  Fwd f = forward_inputs(m, c);
  const ir::TensorType& t = c.input_types[0];
  ir::Value* s = m.op("sigmoid", {f.x[0]});
  ir::Value* one = m.splat(t, 1.0);
  ir::Value* neg = m.splat(t, -1.0);
  ir::Value* ns = m.op("mul", {neg, s});
  ir::Value* oms = m.op("add", {one, ns});
  ir::Value* ss = m.op("mul", {s, oms});
  return m.finish({m.op("mul", {f.gy, ss})});
}

// tanh (reference: src/ops/schemas/elementwise.cpp:550-605): gx = gy * (1 - tanh(x)^2).
Result<ir::Graph> tanh_gradient(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect(c, 1, "1 input"));
  Micro m("tanh_gradient");
  Fwd f = forward_inputs(m, c);
  const ir::TensorType& t = c.input_types[0];
  ir::Value* th = m.op("tanh", {f.x[0]});
  ir::Value* t2 = m.op("mul", {th, th});
  ir::Value* neg = m.splat(t, -1.0);
  ir::Value* nt2 = m.op("mul", {neg, t2});
  ir::Value* one = m.splat(t, 1.0);
  ir::Value* omt = m.op("add", {one, nt2});
  return m.finish({m.op("mul", {f.gy, omt})});
}

// rsqrt (reference: src/ops/schemas/elementwise.cpp:612-660): gx = gy * (-0.5 * r^3), r = rsqrt(x) recomputed.
Result<ir::Graph> rsqrt_gradient(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect(c, 1, "1 input"));
  Micro m("rsqrt_gradient");
  Fwd f = forward_inputs(m, c);
  const ir::TensorType& t = c.input_types[0];
  ir::Value* r = m.op("rsqrt", {f.x[0]});
  ir::Value* r2 = m.op("mul", {r, r});
  ir::Value* r3 = m.op("mul", {r2, r});
  ir::Value* nh = m.splat(t, -0.5);
  ir::Value* coeff = m.op("mul", {nh, r3});
  return m.finish({m.op("mul", {f.gy, coeff})});
}

// gelu (this build's op; no reference counterpart): gx = gelu_grad_internal(x, gy) = gy * (Phi(x) + x * phi(x)).
Result<ir::Graph> gelu_gradient(const NodeContext& c) {
  FRAME_RETURN_IF_ERROR(expect(c, 1, "1 input"));
  Micro m("gelu_gradient");
  Fwd f = forward_inputs(m, c);
  return m.finish({m.op("gelu_grad_internal", {f.x[0], f.gy})});
}

}  // namespace frame::ops::schemas

namespace {
using frame::ir::AttrType;
namespace fs = frame::ops::schemas;
}  // namespace

FRAME_REGISTER_OP("relu_grad_internal")
    .input("x", "relu's original input")
    .input("gy", "upstream gradient of relu's output (same shape/dtype as x)")
    .output("gx", "gy where x > 0, else 0")
    .shape_infer(&fs::infer_relu_grad);

FRAME_REGISTER_OP("matmul_grad_lhs_internal")
    .input("gy", "upstream gradient of matmul's output, rank-2 [m, n]")
    .input("b", "matmul's original rhs, rank-2 [k, n]")
    .output("ga", "gy * b^T, rank-2 [m, k]")
    .shape_infer(&fs::infer_matmul_grad_lhs);

FRAME_REGISTER_OP("matmul_grad_rhs_internal")
    .input("a", "matmul's original lhs, rank-2 [m, k]")
    .input("gy", "upstream gradient of matmul's output, rank-2 [m, n]")
    .output("gb", "a^T * gy, rank-2 [k, n]")
    .shape_infer(&fs::infer_matmul_grad_rhs);

FRAME_REGISTER_OP("conv2d_grad_input_internal")
    .input("dy", "upstream gradient of conv2d's output, rank-4 [N, Cout, out_h, out_w]")
    .input("w", "conv2d's original filter, rank-4 [Cout, Cin/groups, KH, KW]")
    .attr("input_shape", AttrType::kShape, true)
    .attr("stride", AttrType::kInt64Array, true)
    .attr("padding", AttrType::kInt64Array, true)
    .attr("groups", AttrType::kInt64, true)
    .output("gx", "gradient w.r.t. x, rank-4 [N, Cin, H, W]")
    .shape_infer(&fs::infer_conv_grad_input);

FRAME_REGISTER_OP("conv2d_grad_filter_internal")
    .input("x", "conv2d's original input, rank-4 [N, Cin, H, W]")
    .input("dy", "upstream gradient of conv2d's output, rank-4 [N, Cout, out_h, out_w]")
    .attr("filter_shape", AttrType::kShape, true)
    .attr("stride", AttrType::kInt64Array, true)
    .attr("padding", AttrType::kInt64Array, true)
    .attr("groups", AttrType::kInt64, true)
    .output("gw", "gradient w.r.t. w, rank-4 [Cout, Cin/groups, KH, KW]")
    .shape_infer(&fs::infer_conv_grad_filter);

FRAME_REGISTER_OP("max_pool2d_grad_internal")
    .input("dy", "upstream gradient of max_pool2d's output, rank-4 [N, C, out_h, out_w]")
    .input("x", "max_pool2d's original input, rank-4 [N, C, H, W]")
    .attr("input_shape", AttrType::kShape, true)
    .attr("kernel", AttrType::kInt64Array, true)
    .attr("stride", AttrType::kInt64Array, true)
    .attr("padding", AttrType::kInt64Array, true)
    .output("gx", "dy summed into each window's first maximum of x")
    .shape_infer(&fs::infer_max_pool_grad);

FRAME_REGISTER_OP("avg_pool2d_grad_internal")
    .input("dy", "upstream gradient of avg_pool2d's output, rank-4 [N, C, out_h, out_w]")
    .attr("input_shape", AttrType::kShape, true)
    .attr("kernel", AttrType::kInt64Array, true)
    .attr("stride", AttrType::kInt64Array, true)
    .attr("padding", AttrType::kInt64Array, true)
    .output("gx", "dy / (KH*KW) summed over each covering window")
    .shape_infer(&fs::infer_avg_pool_grad);

FRAME_REGISTER_OP("sum")
    .input("x", "input tensor")
    .attr("axes", AttrType::kInt64Array, true)
    .attr("keepdims", AttrType::kBool, false)
    .output("out", "sum of x over axes (every axis when axes is empty)")
    .shape_infer(&fs::infer_sum)
    .gradient(&fs::sum_gradient);

FRAME_REGISTER_OP("sum_grad_internal")
    .input("gy", "upstream gradient of sum's output")
    .attr("input_shape", AttrType::kShape, true)
    .attr("axes", AttrType::kInt64Array, true)
    .output("gx", "gy broadcast back to input_shape along axes")
    .shape_infer(&fs::infer_sum_grad);

FRAME_REGISTER_OP("mse_loss")
    .input("pred", "predicted tensor")
    .input("target", "target tensor")
    .output("out", "mean((pred - target)^2), rank-0")
    .shape_infer(&fs::infer_mse_loss)
    .gradient(&fs::mse_loss_gradient);

FRAME_REGISTER_OP("mse_loss_grad_internal")
    .input("pred", "mse_loss's first input")
    .input("target", "mse_loss's second input")
    .input("gy", "upstream gradient of mse_loss's scalar output")
    .output("gpred", "2 * gy / numel * (pred - target)")
    .shape_infer(&fs::infer_mse_loss_grad);

FRAME_REGISTER_OP("gelu_grad_internal")
    .input("x", "gelu's original input")
    .input("gy", "upstream gradient of gelu's output (same shape/dtype as x)")
    .output("gx", "gy * (Phi(x) + x * phi(x)), the derivative of 0.5 x (1 + erf(x / sqrt 2))")
    .shape_infer(&fs::infer_relu_grad);

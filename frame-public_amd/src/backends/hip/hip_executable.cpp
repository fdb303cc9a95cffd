// HipExecutable and the backend-internal lowering done by HipBackend::compile.
//
// Executor (design analog replaced: src/backends/cuda/cuda_executable.cpp:41-128, which allocates the arena
// and every graph output per run and copies outputs device-to-device afterwards):
//  * the arena is allocated once per stream and reused by later runs on that stream;
//  * steps that produce a graph output write straight into the caller's output tensor;
//  * constants are materialised on the device once, at compile time.
//
// Lowering (allowed inside Backend::compile by the HAL contract, include/frame/hal/backend.h:45-63):
//  * attention (every opt_level): the per-(batch, head) decomposition of multi-head attention becomes one
// attention node (see lower_attention);
//  * epilogue fusion (opt_level >= 1): a matmul
// or conv2d whose only consumer is an elementwise node (add, mul, relu, square, gelu or a fused chain) that
// takes the contraction result as its first operand is replaced by one internal node that applies the
// consumer's program in the contraction's epilogue. The epilogue rounds to the storage dtype after the
// product and after every segment, exactly as the unfused consumer does. The fused matmul also carries
// any_order = 1: small problems may then sum k in a reassociated order (the split-k kernel), within the fp32
// tolerance; opt_level 0 keeps the sequential order, bit-identical to the reference CPU kernel.
//  * grouped GEMMs (opt_level >= 1): 16-bit matmuls (fused or not) that read the same A with equal B shapes,
// output types and epilogue programs (the Q/K/V projections of an attention block) become one grouped node
// launched as one kernel (see lower_grouped_gemms).
//  * GEMM + softmax (opt_level >= 1): a softmax over the rows of a fused matmul of at most 16 columns runs in
// the GEMM's launch (see lower_gemm_softmax).
//  * channels-last conv (every opt_level): a conv that the MFMA implicit-GEMM path accepts becomes
// channels_last(x), channels_last(w) and conv2d_nhwc (see lower_convs); activations whose every use takes
// channels-last data stay channels-last between convs (see plan_channels_last).
// The rewrites run on a private copy of the graph before planning, so the memory plan sees the real lifetimes.
#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <optional>
#include <string>
#include <string_view>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

#include <frame/ir/graph.h>
#include <frame/ops/constant_utils.h>
#include <frame/ops/executable_plan.h>
#include <frame/ops/fused_elementwise_utils.h>
#include <frame/ops/op_registry.h>

#include "hip_backend.h"

namespace frame::backends::hip {

namespace {

template <typename T>
const T* attr_of(const ir::Node* n, const char* key) {
  auto it = n->attrs().find(key);
  return it == n->attrs().end() ? nullptr : std::get_if<T>(&it->second);
}

// Consumer program as fh_ew_op codes, or empty when the consumer cannot become an epilogue.
// `operand_index` is the position of the contraction result among the consumer's inputs.
std::vector<int64_t> epilogue_program(const ir::Node* consumer, size_t operand_index) {
  std::vector<int64_t> codes;
  if (consumer->op() == ops::kFusedElementwiseOpName) {
    ops::FusedElementwiseChain chain;
    if (!ops::decode_and_validate_fused_chain(consumer->attrs(), static_cast<int64_t>(consumer->inputs().size()), chain)
             .is_ok())
      return {};
    for (size_t i = 0; i < chain.sub_ops.size(); ++i) {
      const uint8_t c = ew_code(chain.sub_ops[i]);
      if (c == 0 || chain.arities[i] > 2) return {};
      codes.push_back(c);
    }
    if (chain.arities[0] != (FH_EW_ADD == codes[0] || FH_EW_MUL == codes[0] ? 2 : 1)) return {};
  } else {
    const uint8_t c = ew_code(consumer->op());
    if (c == 0) return {};
    codes.push_back(c);
  }
  // The result must feed segment 0's first operand; add/mul are commutative, so the second slot also works.
  if (operand_index == 0) return codes;
  if (operand_index == 1 && (codes[0] == FH_EW_ADD || codes[0] == FH_EW_MUL)) return codes;
  return {};
}

// relu_grad_internal(x, gy) keeps gy where x > 0. Where the graph also computes r = relu(x), r > 0 exactly where
// x > 0 (relu keeps every x > 0 and maps the rest, NaN included, to zero, -0 or NaN, none of which is > 0), so
// relu_grad(r, gy) is the same tensor bit for bit and x loses a use: a conv or matmul (or the residual add after it)
// whose result fed only the relu and its gradient can then take the relu into its epilogue, and a training graph's
// forward fuses as the inference graph's does.
Status lower_relu_grads(ir::Graph& g) {
  std::unordered_map<const ir::Value*, ir::Value*> relu_of;  // x -> relu(x)
  for (ir::Node* n : g.topological_order())
    if (n->op() == "relu" && n->inputs().size() == 1 && n->outputs().size() == 1 &&
        n->outputs()[0].type().dtype == n->inputs()[0]->type().dtype)
      relu_of.emplace(n->inputs()[0], n->output(0));
  if (relu_of.empty()) return Status::ok();
  const std::vector<ir::Node*> snapshot = g.topological_order();
  for (ir::Node* n : snapshot) {
    if (n->op() != "relu_grad_internal" || n->inputs().size() != 2 || n->outputs().size() != 1) continue;
    auto it = relu_of.find(n->inputs()[0]);
    if (it == relu_of.end() || !(it->second->type().shape == n->inputs()[0]->type().shape)) continue;
    Result<ir::Node*> r = g.create_node(std::string(n->op()), {it->second, n->inputs()[1]}, {n->outputs()[0].type()});
    if (!r.is_ok()) return r.status();
    for (const auto& [k, a] : n->attrs()) r.value()->set_attr(k, a);
    FRAME_RETURN_IF_ERROR(g.replace_all_uses(n->output(0), r.value()->output(0)));
    FRAME_RETURN_IF_ERROR(g.erase_node(n));
  }
  return Status::ok();
}

// relu_grad_internal(x, m) with m = max_pool2d_grad_internal(dy, x) used only there (the stem of a training graph
// after lower_relu_grads, x the pool's input and the relu's output) becomes one kMaxPoolReluGradOp node: the pool
// gradient kernel already holds x where it writes dx, so the mask costs no pass of its own.
Status lower_pool_relu_grads(ir::Graph& g) {
  std::unordered_map<const ir::Value*, int> uses;
  for (const ir::Node* n : g.topological_order())
    for (const ir::Value* v : n->inputs()) ++uses[v];
  for (const ir::Value* v : g.outputs()) uses[v] += 1000;
  const std::vector<ir::Node*> snapshot = g.topological_order();
  for (ir::Node* n : snapshot) {
    if (n->op() != "relu_grad_internal" || n->inputs().size() != 2 || n->outputs().size() != 1) continue;
    ir::Value* m = n->inputs()[1];
    ir::Node* p = m->producer();
    if (p == nullptr || p->op() != "max_pool2d_grad_internal" || p->inputs().size() != 2 || uses[m] != 1) continue;
    if (p->inputs()[1] != n->inputs()[0] || !(p->outputs()[0].type().dtype == n->outputs()[0].type().dtype)) continue;
    Result<ir::Node*> f = g.create_node(std::string(kMaxPoolReluGradOp), {p->inputs()[0], p->inputs()[1]},
                                        {n->outputs()[0].type()});
    if (!f.is_ok()) return f.status();
    for (const auto& [k, a] : p->attrs()) f.value()->set_attr(k, a);
    FRAME_RETURN_IF_ERROR(g.replace_all_uses(n->output(0), f.value()->output(0)));
    FRAME_RETURN_IF_ERROR(g.erase_node(n));
    FRAME_RETURN_IF_ERROR(g.erase_node(p));
  }
  return Status::ok();
}

// relu_grad_internal(x, s) with s = add(a, b) used only there (a residual block's gradient: the sum of its two
// consumers' gradients, then the block relu's mask) becomes one kEwProgramOp node [add, FH_EW_RELU_MASK] over
// (a, b, x): the sum is rounded as the add node stores it and masked as relu_grad does, bit for bit, in one pass.
Status lower_masked_adds(ir::Graph& g) {
  std::unordered_map<const ir::Value*, int> uses;
  for (const ir::Node* n : g.topological_order())
    for (const ir::Value* v : n->inputs()) ++uses[v];
  for (const ir::Value* v : g.outputs()) uses[v] += 1000;
  const std::vector<ir::Node*> snapshot = g.topological_order();
  for (ir::Node* n : snapshot) {
    if (n->op() != "relu_grad_internal" || n->inputs().size() != 2 || n->outputs().size() != 1) continue;
    ir::Value* s = n->inputs()[1];
    ir::Node* p = s->producer();
    if (p == nullptr || p->op() != "add" || p->inputs().size() != 2 || uses[s] != 1) continue;
    const ir::TensorType& t = n->outputs()[0].type();
    bool same = true;
    for (const ir::Value* v : {p->inputs()[0], p->inputs()[1], n->inputs()[0], s})
      same = same && v->type().dtype == t.dtype && v->type().shape == t.shape;
    if (!same) continue;
    Result<ir::Node*> f = g.create_node(std::string(kEwProgramOp), {p->inputs()[0], p->inputs()[1], n->inputs()[0]}, {t});
    if (!f.is_ok()) return f.status();
    f.value()->set_attr("ew_ops", ir::AttrValue{std::vector<int64_t>{FH_EW_ADD, FH_EW_RELU_MASK}});
    FRAME_RETURN_IF_ERROR(g.replace_all_uses(n->output(0), f.value()->output(0)));
    FRAME_RETURN_IF_ERROR(g.erase_node(n));
    FRAME_RETURN_IF_ERROR(g.erase_node(p));
  }
  return Status::ok();
}

// A matmul or conv2d whose result's only use is an elementwise program (a single add/mul/relu/square/gelu node or a
// fused chain of them) becomes one epilogue node; a second single-use elementwise consumer of that node's result
// extends its program (conv -> add -> relu of a training graph, whose add and relu the fusion pass left apart while
// the add's result also fed relu_grad, becomes the add;relu epilogue of the inference graph).
Status lower_epilogues(ir::Graph& g) {
  std::unordered_map<const ir::Value*, int> uses;
  for (const ir::Node* n : g.topological_order())
    for (const ir::Value* v : n->inputs()) ++uses[v];
  for (const ir::Value* v : g.outputs()) uses[v] += 1000;  // graph outputs are never folded away
  const std::vector<ir::Node*> snapshot = g.topological_order();
  // snapshot nodes fused away (checked only against snapshot nodes: an epilogue node created here may reuse the
  // address of one erased before it; a producer reached through a live consumer's input is always live)
  std::unordered_set<const ir::Node*> erased;
  for (ir::Node* c : snapshot) {
    if (erased.count(c) || c->outputs().size() != 1) continue;
    for (size_t idx = 0; idx < std::min<size_t>(2, c->inputs().size()); ++idx) {
      ir::Value* v = c->inputs()[idx];
      ir::Node* p = v->producer();
      if (p == nullptr || uses[v] != 1) continue;
      const bool chained = p->op() == kGemmEpilogueOp || p->op() == kConvEpilogueOp;
      const bool is_mm = p->op() == "matmul" || p->op() == kGemmEpilogueOp;
      const bool is_conv = p->op() == "conv2d" || p->op() == kConvEpilogueOp;
      if (!is_mm && !is_conv) continue;
      if (!(p->outputs()[0].type().dtype == c->outputs()[0].type().dtype)) continue;
      std::vector<int64_t> prog = epilogue_program(c, idx);
      size_t n_main = p->inputs().size();
      if (chained) {
        const auto* before = attr_of<std::vector<int64_t>>(p, "ep_ops");
        const auto* main = attr_of<int64_t>(p, "n_main_inputs");
        if (before == nullptr || main == nullptr || prog.empty()) continue;
        prog.insert(prog.begin(), before->begin(), before->end());
        n_main = static_cast<size_t>(*main);
      }
      if (prog.empty() || prog.size() > FH_MAX_SEGMENTS) continue;
      std::vector<ir::Value*> ins(p->inputs().begin(), p->inputs().end());
      for (size_t j = 0; j < c->inputs().size(); ++j)
        if (j != idx) ins.push_back(c->inputs()[j]);
      if (ins.size() - n_main > FH_MAX_SEGMENTS) continue;
      Result<ir::Node*> f = g.create_node(std::string(is_mm ? kGemmEpilogueOp : kConvEpilogueOp), ins,
                                          {c->outputs()[0].type()});
      if (!f.is_ok()) return f.status();
      for (const auto& [k, a] : p->attrs()) f.value()->set_attr(k, a);
      f.value()->set_attr("ep_ops", ir::AttrValue{prog});
      f.value()->set_attr("n_main_inputs", ir::AttrValue{static_cast<int64_t>(n_main)});
      if (is_mm) f.value()->set_attr("any_order", ir::AttrValue{int64_t{1}});
      uses[f.value()->output(0)] = uses[c->output(0)];
      FRAME_RETURN_IF_ERROR(g.replace_all_uses(c->output(0), f.value()->output(0)));
      FRAME_RETURN_IF_ERROR(g.erase_node(c));
      FRAME_RETURN_IF_ERROR(g.erase_node(p));
      erased.insert(c);
      erased.insert(p);
      break;
    }
  }
  return Status::ok();
}

int32_t conv_dtype_code(const ir::TensorType& t);

// A 7x7 stride-2 convolution (plain conv2d, or a conv epilogue node whose program is relu alone) whose result's only
// use is a 3x3 stride-2 max_pool2d, directly or through a relu whose only use is the pool, becomes one
// kConvStemPoolOp node that produces the pool's output (fh_conv2d_stem_pool takes the geometry): ResNet's stem
// without its 4x larger convolution output ever reaching memory. Runs at every opt level, like the conv lowering.
Status lower_stem_pools(ir::Graph& g) {
  std::unordered_map<const ir::Value*, int> uses;
  for (const ir::Node* n : g.topological_order())
    for (const ir::Value* v : n->inputs()) ++uses[v];
  for (const ir::Value* v : g.outputs()) uses[v] += 1000;  // graph outputs are never folded away
  const std::vector<ir::Node*> snapshot = g.topological_order();
  std::unordered_set<const ir::Node*> erased;
  for (ir::Node* pool : snapshot) {
    if (erased.count(pool) || pool->op() != "max_pool2d" || pool->inputs().size() != 1 || pool->outputs().size() != 1)
      continue;
    ir::Value* v = pool->inputs()[0];
    ir::Node* p = v->producer();
    if (p == nullptr || uses[v] != 1) continue;
    ir::Node* relu_node = nullptr;
    if (p->op() == "relu" && p->inputs().size() == 1) {
      relu_node = p;
      v = p->inputs()[0];
      p = v->producer();
      if (p == nullptr || uses[v] != 1) continue;
    }
    bool relu = relu_node != nullptr;
    size_t n_main = p->inputs().size();
    if (p->op() == kConvEpilogueOp) {
      const auto* prog = attr_of<std::vector<int64_t>>(p, "ep_ops");
      const auto* nm = attr_of<int64_t>(p, "n_main_inputs");
      if (prog == nullptr || *prog != std::vector<int64_t>{FH_EW_RELU} || nm == nullptr) continue;
      n_main = static_cast<size_t>(*nm);
      relu = true;  // relu(relu(x)) == relu(x)
    } else if (p->op() != "conv2d") {
      continue;
    }
    if ((n_main != 2 && n_main != 3) || n_main != p->inputs().size()) continue;
    const auto* stride = attr_of<std::vector<int64_t>>(p, "stride");
    const auto* pad = attr_of<std::vector<int64_t>>(p, "padding");
    const auto* groups = attr_of<int64_t>(p, "groups");
    const auto* pk = attr_of<std::vector<int64_t>>(pool, "kernel");
    const auto* ps = attr_of<std::vector<int64_t>>(pool, "stride");
    const auto* pp = attr_of<std::vector<int64_t>>(pool, "padding");
    if (stride == nullptr || pad == nullptr || groups == nullptr || pk == nullptr || ps == nullptr || pp == nullptr ||
        stride->size() != 2 || pad->size() != 2 || pk->size() != 2 || ps->size() != 2 || pp->size() != 2)
      continue;
    const ir::TensorType& xt = p->inputs()[0]->type();
    const ir::TensorType& wt = p->inputs()[1]->type();
    const ir::TensorType& yt = pool->outputs()[0].type();
    if (xt.shape.rank() != 4 || wt.shape.rank() != 4 || !(xt.dtype == yt.dtype) || !(wt.dtype == yt.dtype)) continue;
    const int64_t geom[12] = {xt.shape.dim(0), xt.shape.dim(1), xt.shape.dim(2), xt.shape.dim(3), wt.shape.dim(0),
                              wt.shape.dim(2),  wt.shape.dim(3),  (*stride)[0],    (*stride)[1],    (*pad)[0],
                              (*pad)[1],        *groups};
    const int64_t pgeom[6] = {(*pk)[0], (*pk)[1], (*ps)[0], (*ps)[1], (*pp)[0], (*pp)[1]};
    if (wt.shape.dim(1) != geom[1] || fh_conv2d_stem_pool_supported(conv_dtype_code(yt), geom, pgeom) == 0) continue;
    std::vector<ir::Value*> ins(p->inputs().begin(), p->inputs().end());
    Result<ir::Node*> f = g.create_node(std::string(kConvStemPoolOp), ins, {yt});
    if (!f.is_ok()) return f.status();
    f.value()->set_attr("stride", ir::AttrValue{*stride});
    f.value()->set_attr("padding", ir::AttrValue{*pad});
    f.value()->set_attr("groups", ir::AttrValue{*groups});
    f.value()->set_attr("kernel", ir::AttrValue{*pk});
    f.value()->set_attr("pool_stride", ir::AttrValue{*ps});
    f.value()->set_attr("pool_padding", ir::AttrValue{*pp});
    f.value()->set_attr("relu", ir::AttrValue{static_cast<int64_t>(relu ? 1 : 0)});
    FRAME_RETURN_IF_ERROR(g.replace_all_uses(pool->output(0), f.value()->output(0)));
    FRAME_RETURN_IF_ERROR(g.erase_node(pool));
    erased.insert(pool);
    if (relu_node != nullptr) {
      FRAME_RETURN_IF_ERROR(g.erase_node(relu_node));
      erased.insert(relu_node);
    }
    FRAME_RETURN_IF_ERROR(g.erase_node(p));
    erased.insert(p);
  }
  return Status::ok();
}

int32_t conv_dtype_code(const ir::TensorType& t) {
  return t.dtype.code() == DTypeCode::kBFloat16  ? FH_BF16
         : t.dtype.code() == DTypeCode::kFloat16 ? FH_F16
         : t.dtype.code() == DTypeCode::kFloat32 ? FH_F32
                                                 : -1;
}

// Whether the channels-last MFMA path takes conv node `n` (conv2d or conv epilogue), with its geometry
// {N, Cin, H, W, Cout, KH, KW, sh, sw, ph, pw, groups} and whether it goes through the C8 layout (Cin <= 8, 16-bit).
struct ConvLowering {
  bool ok = false;
  bool c8 = false;
  int64_t geom[12] = {};
};

ConvLowering plan_conv(const ir::Node* n) {
  ConvLowering p;
  const bool is_conv = n->op() == "conv2d" || n->op() == kConvEpilogueOp;
  if (!is_conv || n->outputs().size() != 1 || n->inputs().size() < 2) return p;
  const ir::TensorType& xt = n->inputs()[0]->type();
  const ir::TensorType& wt = n->inputs()[1]->type();
  auto get = [&](const char* k) -> const ir::AttrValue* {
    auto it = n->attrs().find(k);
    return it == n->attrs().end() ? nullptr : &it->second;
  };
  const auto* stride = get("stride") ? std::get_if<std::vector<int64_t>>(get("stride")) : nullptr;
  const auto* pad = get("padding") ? std::get_if<std::vector<int64_t>>(get("padding")) : nullptr;
  const auto* groups = get("groups") ? std::get_if<int64_t>(get("groups")) : nullptr;
  const int32_t dt = xt.dtype.code() == DTypeCode::kBFloat16  ? FH_BF16
                     : xt.dtype.code() == DTypeCode::kFloat16 ? FH_F16
                     : xt.dtype.code() == DTypeCode::kFloat32 ? FH_F32
                                                              : -1;
  if (!stride || !pad || !groups || stride->size() != 2 || pad->size() != 2 || dt < 0 || xt.shape.rank() != 4 ||
      wt.shape.rank() != 4 || !(wt.dtype == xt.dtype) || wt.shape.dim(1) != xt.shape.dim(1))
    return p;
  const int64_t geom[12] = {xt.shape.dim(0), xt.shape.dim(1), xt.shape.dim(2), xt.shape.dim(3),
                            wt.shape.dim(0), wt.shape.dim(2), wt.shape.dim(3), (*stride)[0],
                            (*stride)[1],    (*pad)[0],       (*pad)[1],       *groups};
  // Cin <= 8 goes through the C8 layout (channels padded to 8, four filter positions per k-stage)
  p.c8 = xt.shape.dim(1) <= 8 && *groups == 1 && dt != FH_F32;
  int64_t geom_k[12];
  std::copy(geom, geom + 12, geom_k);
  if (p.c8) geom_k[1] = 8;
  std::copy(geom, geom + 12, p.geom);
  p.ok = fh_conv2d_nhwc_supported(dt, geom_k) == 1;
  return p;
}

// conv2d_grad_input_internal(dy, w) as dx = conv(dilate(dy, stride), flip(w)) with stride 1 and padding
// KH-1-pad on the implicit-GEMM kernel: the transposed convolution. dy is dilated to Hu = (Ho-1)*s + 1 + r rows,
// r = (H + 2 pad - KH) mod s (the rows the forward's floor dropped), so the output is exactly [N,Cin,H,W]. Only
// groups == 1 and pad <= K-1, and geometries the kernel takes; others keep the direct kernel.
struct GradInputLowering {
  bool ok = false;
  int64_t n = 0, cout = 0, cin = 0, hu = 0, wu = 0, kh = 0, kw = 0, sh = 1, sw = 1, ph = 0, pw = 0;
};

GradInputLowering plan_grad_input(const ir::Node* n) {
  GradInputLowering g;
  if (n->op() != "conv2d_grad_input_internal" || n->inputs().size() != 2) return g;
  const ir::TensorType& dy = n->inputs()[0]->type();
  const ir::TensorType& w = n->inputs()[1]->type();
  auto get = [&](const char* k) -> const ir::AttrValue* {
    auto it = n->attrs().find(k);
    return it == n->attrs().end() ? nullptr : &it->second;
  };
  const auto* xs = get("input_shape") ? std::get_if<Shape>(get("input_shape")) : nullptr;
  const auto* stride = get("stride") ? std::get_if<std::vector<int64_t>>(get("stride")) : nullptr;
  const auto* pad = get("padding") ? std::get_if<std::vector<int64_t>>(get("padding")) : nullptr;
  const auto* groups = get("groups") ? std::get_if<int64_t>(get("groups")) : nullptr;
  const int32_t dt = dy.dtype.code() == DTypeCode::kBFloat16  ? FH_BF16
                     : dy.dtype.code() == DTypeCode::kFloat16 ? FH_F16
                     : dy.dtype.code() == DTypeCode::kFloat32 ? FH_F32
                                                              : -1;
  if (!xs || !stride || !pad || !groups || stride->size() != 2 || pad->size() != 2 || *groups != 1 || dt < 0 ||
      xs->rank() != 4 || dy.shape.rank() != 4 || w.shape.rank() != 4)
    return g;
  g.n = xs->dim(0), g.cin = xs->dim(1), g.cout = w.shape.dim(0), g.kh = w.shape.dim(2), g.kw = w.shape.dim(3);
  g.sh = (*stride)[0], g.sw = (*stride)[1], g.ph = (*pad)[0], g.pw = (*pad)[1];
  if (g.sh < 1 || g.sw < 1 || g.ph > g.kh - 1 || g.pw > g.kw - 1) return g;
  const int64_t eh = xs->dim(2) + 2 * g.ph - g.kh, ew = xs->dim(3) + 2 * g.pw - g.kw;
  if (eh < 0 || ew < 0) return g;
  g.hu = (dy.shape.dim(2) - 1) * g.sh + 1 + eh % g.sh;
  g.wu = (dy.shape.dim(3) - 1) * g.sw + 1 + ew % g.sw;
  const int64_t geom[12] = {g.n, g.cout, g.hu, g.wu, g.cin, g.kh, g.kw, 1, 1, g.kh - 1 - g.ph, g.kw - 1 - g.pw, 1};
  // the transposed conv's input channels are the forward's Cout: the plain (not C8) channels-last layout only
  g.ok = g.cout % (dt == FH_F32 ? 16 : 32) == 0 && fh_conv2d_nhwc_supported(dt, geom) == 1;
  return g;
}

// conv2d_grad_filter_internal(x, dy) on the MFMA filter-gradient kernel: x channels-last (the C8 pack when
// Cin <= 8), dy channels-last, plus the kernel's split-K workspace as a second, planned output.
struct GradFilterLowering {
  bool ok = false, c8 = false;
  int64_t workspace = 0;
};

GradFilterLowering plan_grad_filter(const ir::Node* n) {
  GradFilterLowering g;
  if (n->op() != "conv2d_grad_filter_internal" || n->inputs().size() != 2) return g;
  const ir::TensorType& x = n->inputs()[0]->type();
  const ir::TensorType& dy = n->inputs()[1]->type();
  auto get = [&](const char* k) -> const ir::AttrValue* {
    auto it = n->attrs().find(k);
    return it == n->attrs().end() ? nullptr : &it->second;
  };
  const auto* ws = get("filter_shape") ? std::get_if<Shape>(get("filter_shape")) : nullptr;
  const auto* stride = get("stride") ? std::get_if<std::vector<int64_t>>(get("stride")) : nullptr;
  const auto* pad = get("padding") ? std::get_if<std::vector<int64_t>>(get("padding")) : nullptr;
  const auto* groups = get("groups") ? std::get_if<int64_t>(get("groups")) : nullptr;
  const int32_t dt = x.dtype.code() == DTypeCode::kBFloat16 ? FH_BF16 : x.dtype.code() == DTypeCode::kFloat16 ? FH_F16 : -1;
  if (!ws || !stride || !pad || !groups || stride->size() != 2 || pad->size() != 2 || dt < 0 || x.shape.rank() != 4 ||
      dy.shape.rank() != 4 || ws->rank() != 4)
    return g;
  const int64_t geom[12] = {x.shape.dim(0), x.shape.dim(1), x.shape.dim(2), x.shape.dim(3), ws->dim(0), ws->dim(2),
                            ws->dim(3),     (*stride)[0],   (*stride)[1],   (*pad)[0],      (*pad)[1],  *groups};
  g.c8 = x.shape.dim(1) <= 8;
  const int64_t cin_pad = g.c8 ? 8 : x.shape.dim(1);
  if (!g.c8 && cin_pad % 8 != 0) return g;
  g.workspace = fh_conv2d_wgrad_workspace(dt, geom, static_cast<int32_t>(cin_pad), nullptr);
  g.ok = g.workspace > 0;
  return g;
}

// Channels-last activations between convolutions. Values that must share a layout form groups (union-find):
// an elementwise node's rank-4 operands and result, a pool's input and output, a lowered conv's result and its
// epilogue operands. A group is kept channels-last ([N,H,W,C] in the lowered graph) when every member is produced
// by a lowered conv, a pool or an elementwise node, and every use is one that takes channels-last data: input 0
// of a lowered non-C8 conv, a conv epilogue operand, a pool, an elementwise node, or a reshape of a 1x1 plane
// (the same bytes in either layout). Graph inputs and outputs stay NCHW, so nothing outside the backend sees it.
// A rank-4 `sum` whose input can be channels-last: without keepdims, and with its kept axes in the same order in
// both layouts (NCHW axis 0,1,2,3 is NHWC axis 0,3,1,2), so the output is the same tensor. Returns the axes for
// the channels-last input.
std::optional<std::vector<int64_t>> nhwc_sum_axes(const ir::Node* n) {
  if (n->op() != "sum" || n->inputs()[0]->type().shape.rank() != 4) return std::nullopt;
  const auto* axes = attr_of<std::vector<int64_t>>(n, "axes");
  const auto* kd = attr_of<bool>(n, "keepdims");
  if (axes == nullptr || (kd != nullptr && *kd)) return std::nullopt;
  static constexpr int64_t to_nhwc[4] = {0, 3, 1, 2};
  bool reduced[4] = {axes->empty(), axes->empty(), axes->empty(), axes->empty()};
  for (int64_t a : *axes) {
    if (a < 0 || a > 3) return std::nullopt;
    reduced[a] = true;
  }
  int64_t last = -1;
  std::vector<int64_t> out;
  for (int64_t a = 0; a < 4; ++a) {
    if (reduced[a]) {
      out.push_back(to_nhwc[a]);
      continue;
    }
    if (to_nhwc[a] < last) return std::nullopt;
    last = to_nhwc[a];
  }
  std::sort(out.begin(), out.end());
  return out;
}

// A conv the band kernel takes when its activation, output and residual operand are NCHW and its filter stays in
// the graph's [Cout][Cin][KH][KW] layout (fh_conv2d_w_oihw_supported on its geometry and epilogue program).
bool band_conv(const ir::Node* n, const ConvLowering& p) {
  if (!p.ok || p.c8) return false;
  fh_epilogue qe{};
  if (const auto* prog = attr_of<std::vector<int64_t>>(n, "ep_ops")) {
    if (prog->size() > FH_MAX_SEGMENTS) return false;
    qe.nseg = static_cast<int32_t>(prog->size());
    for (size_t s = 0; s < prog->size(); ++s) qe.ops[s] = static_cast<uint8_t>((*prog)[s]);
  }
  return fh_conv2d_w_oihw_supported(conv_dtype_code(n->inputs()[0]->type()), p.geom, &qe) != 0;
}

std::unordered_set<const ir::Value*> plan_channels_last(const ir::Graph& src) {
  std::unordered_map<const ir::Value*, const ir::Value*> parent;
  auto find = [&](const ir::Value* v) {
    const ir::Value* r = v;
    while (parent.count(r) && parent[r] != r) r = parent[r];
    while (parent.count(v) && parent[v] != r) {  // path compression
      const ir::Value* next = parent[v];
      parent[v] = r;
      v = next;
    }
    return r;
  };
  auto add = [&](const ir::Value* v) {
    if (!parent.count(v)) parent[v] = v;
  };
  auto unite = [&](const ir::Value* a, const ir::Value* b) {
    add(a);
    add(b);
    const ir::Value *ra = find(a), *rb = find(b);
    if (ra != rb) parent[ra] = rb;
  };
  auto is_ew = [](const ir::Node* n) {
    return ew_code(n->op()) != 0 || n->op() == ops::kFusedElementwiseOpName || n->op() == "relu_grad_internal" ||
           n->op() == kEwProgramOp;
  };
  auto is_pool = [](const ir::Node* n) { return n->op() == "max_pool2d" || n->op() == "avg_pool2d"; };
  auto rank4 = [](const ir::Value* v) { return v->type().shape.rank() == 4; };
  // training-graph nodes that read or write channels-last operands once lowered
  auto is_grad_input = [](const ir::Node* n) { return plan_grad_input(n).ok; };
  auto is_avg_pool_grad = [](const ir::Node* n) {
    return n->op() == "avg_pool2d_grad_internal" && n->outputs()[0].type().shape.rank() == 4 &&
           n->outputs()[0].type().shape.dim(1) * static_cast<int64_t>(n->outputs()[0].type().dtype.itemsize()) % 16 == 0;
  };

  std::unordered_map<const ir::Value*, std::vector<std::pair<const ir::Node*, size_t>>> uses;
  std::unordered_map<const ir::Node*, ConvLowering> convs;
  for (const ir::Node* n : src.topological_order()) {
    for (size_t i = 0; i < n->inputs().size(); ++i) uses[n->inputs()[i]].push_back({n, i});
    const ConvLowering p = plan_conv(n);
    if (p.ok) {
      convs[n] = p;
      add(&n->outputs()[0]);
      if (n->op() == kConvEpilogueOp) {
        const auto* nm = attr_of<int64_t>(n, "n_main_inputs");
        for (size_t i = nm ? static_cast<size_t>(*nm) : 2; i < n->inputs().size(); ++i)
          unite(&n->outputs()[0], n->inputs()[i]);
      }
    } else if ((is_ew(n) || is_pool(n)) && n->outputs().size() == 1 && rank4(&n->outputs()[0])) {
      add(&n->outputs()[0]);
      for (const ir::Value* in : n->inputs())
        if (rank4(in)) unite(&n->outputs()[0], in);
    } else if (is_grad_input(n)) {
      add(&n->outputs()[0]);
    } else if (is_avg_pool_grad(n)) {
      unite(&n->outputs()[0], n->inputs()[0]);
    } else if (n->op() == "reshape" && rank4(&n->outputs()[0]) && n->outputs()[0].type().shape.dim(2) == 1 &&
               n->outputs()[0].type().shape.dim(3) == 1) {
      add(&n->outputs()[0]);  // [N,C,1,1]: the same bytes in either layout
    }
  }
  std::unordered_set<const ir::Value*> bad;  // group roots that must stay NCHW
  std::unordered_set<const ir::Value*> graph_outputs(src.outputs().begin(), src.outputs().end());
  for (const auto& [v, unused] : parent) {
    (void)unused;
    const ir::Value* root = find(v);
    const ir::Node* p = v->producer();
    const bool plane1 = rank4(v) && v->type().shape.dim(2) == 1 && v->type().shape.dim(3) == 1;
    const bool producer_ok = p != nullptr && (convs.count(p) || is_ew(p) || is_pool(p) || is_grad_input(p) ||
                                              is_avg_pool_grad(p) || (p->op() == "reshape" && plane1));
    bool uses_ok = !graph_outputs.count(v);
    for (const auto& [c, idx] : uses[v]) {
      if (!uses_ok) break;
      if (auto it = convs.find(c); it != convs.end()) {
        const auto* nm = attr_of<int64_t>(c, "n_main_inputs");
        const size_t n_main = c->op() == kConvEpilogueOp ? (nm ? static_cast<size_t>(*nm) : 2) : c->inputs().size();
        uses_ok = (idx == 0 && !it->second.c8) || idx >= n_main;
      } else if (is_ew(c) || is_pool(c)) {
        uses_ok = rank4(&c->outputs()[0]);
      } else if (c->op() == "reshape") {
        const Shape& sh = v->type().shape;
        uses_ok = sh.rank() == 4 && sh.dim(2) == 1 && sh.dim(3) == 1;
      } else if (is_grad_input(c)) {
        uses_ok = idx == 0;  // dy
      } else if (const GradFilterLowering gf = plan_grad_filter(c); gf.ok) {
        uses_ok = idx == 1 || !gf.c8;  // dy, or x when it needs no C8 pack
      } else if (is_avg_pool_grad(c)) {
        uses_ok = true;
      } else if (c->op() == "sum") {
        uses_ok = nhwc_sum_axes(c).has_value();
      } else {
        uses_ok = false;
      }
    }
    if (!producer_ok || !uses_ok || !rank4(v)) bad.insert(root);
  }
  // Forward graphs: a group that a band conv produces stays NCHW when every conv producing into it is a band conv
  // or a C8 stem conv (both write NCHW), so the band kernel (NCHW in and out, the filter read as it is) runs it:
  // ResNet's 56x56 layer, whose channels-last convs took 32-37 us each, against 24-26 us on the band kernel. Its
  // pool runs the NCHW kernel; a non-band conv reading such a value gets one channels-last copy of it.
  bool forward = true;
  for (const ir::Node* n : src.topological_order())
    if (n->op().find("grad") != std::string::npos) forward = false;
  if (forward) {
    std::unordered_map<const ir::Value*, std::pair<bool, bool>> group;  // root -> (band producer, other conv producer)
    for (const auto& [v, unused] : parent) {
      (void)unused;
      const ir::Node* p = v->producer();
      auto it = p != nullptr ? convs.find(p) : convs.end();
      if (it == convs.end()) continue;
      auto& g = group[find(v)];
      if (band_conv(p, it->second)) g.first = true;
      else if (!it->second.c8) g.second = true;
    }
    for (const auto& [root, g] : group)
      if (g.first && !g.second) bad.insert(root);
  }
  std::unordered_set<const ir::Value*> nhwc;
  for (const auto& [v, unused] : parent) {
    (void)unused;
    if (!bad.count(find(v))) nhwc.insert(v);
  }
  return nhwc;
}

// Lowers every conv2d / conv epilogue node that the channels-last MFMA path accepts (fh_conv2d_nhwc_supported)
// to  x_nhwc = channels_last(x); w_khwc = channels_last(w); y = conv2d_nhwc(x_nhwc, w_khwc, bias?, ep...).
// The filters that are graph inputs (weights fed per run) are transposed together by one
// channels_last_multi node, emitted before the first conv that needs one, instead of one launch per layer.
// The graph is rebuilt in topological order with the new nodes emitted in the conv's place, so the transposed
// operands become ordinary intermediates that the memory plan places and recycles.
Result<ir::Graph> lower_convs(const ir::Graph& src) {
  std::unordered_map<const ir::Value*, ir::Value*> map;
  ir::Graph out{std::string(src.name())};
  const std::unordered_set<const ir::Value*> nhwc = plan_channels_last(src);
  // the lowered graph's type of a source value: [N,H,W,C] when it is kept channels-last
  auto lowered_type = [&](const ir::Value* v) {
    ir::TensorType t = v->type();
    if (nhwc.count(v)) {
      const Shape& s = t.shape;
      t.shape = Shape({s.dim(0), s.dim(2), s.dim(3), s.dim(1)});
    }
    return t;
  };
  auto channels_last_type = [](const ir::Value* v) {
    ir::TensorType t = v->type();
    const Shape& s = t.shape;
    t.shape = Shape({s.dim(0), s.dim(2), s.dim(3), s.dim(1)});
    return t;
  };
  // A channels-last pool to a 1x1 plane whose only use is a reshape to [N, C] (ResNet's global pool before the
  // FC): [N,1,1,C] and [N,C] are the same bytes, so the pool writes the reshape's type and the reshape (a device
  // copy and a launch) goes away.
  std::unordered_map<const ir::Node*, const ir::Node*> reshaped_pool;  // pool -> its reshape
  std::unordered_set<const ir::Node*> folded_reshape;
  {
    std::unordered_map<const ir::Value*, int> n_uses;
    for (const ir::Node* n : src.topological_order())
      for (const ir::Value* in : n->inputs()) ++n_uses[in];
    std::unordered_set<const ir::Value*> outs(src.outputs().begin(), src.outputs().end());
    for (const ir::Node* r : src.topological_order()) {
      if (r->op() != "reshape" || r->inputs().size() != 1 || r->outputs().size() != 1) continue;
      const ir::Value* v = r->inputs()[0];
      const ir::Node* p = v->producer();
      if (p == nullptr || (p->op() != "max_pool2d" && p->op() != "avg_pool2d") || p->outputs().size() != 1) continue;
      const Shape& vs = v->type().shape;
      const Shape& rs = r->outputs()[0].type().shape;
      if (!nhwc.count(v) || outs.count(v) || n_uses[v] != 1 || vs.rank() != 4 || vs.dim(2) != 1 || vs.dim(3) != 1 ||
          rs.rank() != 2 || rs.dim(0) != vs.dim(0) || rs.dim(1) != vs.dim(1) || nhwc.count(&r->outputs()[0]))
        continue;
      reshaped_pool[p] = r;
      folded_reshape.insert(r);
    }
  }
  std::unordered_map<const ir::Value*, ir::Value*> cl_copies;  // one channels-last copy per value
  // one C8 pack per value (a training graph's stem input feeds both the conv and its filter gradient)
  std::unordered_map<const ir::Value*, ir::Value*> c8_packs;
  auto pack_c8 = [&](ir::Value* v) -> Result<ir::Value*> {
    if (auto it = c8_packs.find(v); it != c8_packs.end()) return it->second;
    ir::TensorType tx = v->type();
    const Shape& xs = tx.shape;
    tx.shape = Shape({xs.dim(0), xs.dim(2), xs.dim(3), 8});
    Result<ir::Node*> px = out.create_node(std::string(kPackInputC8Op), {v}, {tx});
    if (!px.is_ok()) return px.status();
    c8_packs[v] = px.value()->output(0);
    return px.value()->output(0);
  };
  auto channels_last = [&](ir::Value* v) -> Result<ir::Value*> {
    if (auto it = cl_copies.find(v); it != cl_copies.end()) return it->second;
    Result<ir::Node*> n = out.create_node(std::string(kChannelsLastOp), {v}, {channels_last_type(v)});
    if (!n.is_ok()) return n.status();
    cl_copies[v] = n.value()->output(0);
    return n.value()->output(0);
  };

  // Whether a lowered conv reads its NCHW activation (FH_CONV_IN_NCHW) and, writing NCHW, takes its filter in the
  // graph's own [Cout][Cin][KH][KW] layout too (FH_CONV_W_OIHW, the band kernel): then neither operand is copied.
  auto reads_nchw = [&](const ir::Node* n, const ConvLowering& p) {
    return p.ok && !p.c8 && !nhwc.count(n->inputs()[0]) &&
           fh_conv2d_nchw_in_supported(conv_dtype_code(n->inputs()[0]->type()), p.geom) != 0;
  };
  auto takes_oihw = [&](const ir::Node* n, const ConvLowering& p) {
    if (!reads_nchw(n, p) || nhwc.count(&n->outputs()[0])) return false;
    fh_epilogue qe{};
    if (const auto* prog = attr_of<std::vector<int64_t>>(n, "ep_ops")) {
      if (prog->size() > FH_MAX_SEGMENTS) return false;
      qe.nseg = static_cast<int32_t>(prog->size());
      for (size_t s = 0; s < prog->size(); ++s) qe.ops[s] = static_cast<uint8_t>((*prog)[s]);
    }
    return fh_conv2d_w_oihw_supported(conv_dtype_code(n->inputs()[0]->type()), p.geom, &qe) != 0;
  };

  // graph-input filters of the non-C8 lowered convs that need a channels-last copy, in first-use order, each once
  std::vector<const ir::Value*> batched;
  {
    std::unordered_set<const ir::Value*> seen;
    for (const ir::Node* n : src.topological_order()) {
      const ConvLowering p = plan_conv(n);
      const ir::Value* w = p.ok && !p.c8 && !takes_oihw(n, p) ? n->inputs()[1] : nullptr;
      if (w == nullptr || w->producer() == nullptr || w->producer()->op() != ir::kGraphInputOp || seen.count(w)) continue;
      if (w->type().shape.dim(1) * w->type().shape.dim(2) * w->type().shape.dim(3) > kMultiPlaneMax) continue;
      seen.insert(w);
      batched.push_back(w);
    }
  }
  std::unordered_map<const ir::Value*, ir::Value*> batched_out;  // source filter -> its transposed value
  bool batched_emitted = false;
  auto emit_batched = [&]() -> Status {
    batched_emitted = true;
    std::vector<const ir::Value*> ready;
    for (const ir::Value* w : batched)
      if (map.count(w)) ready.push_back(w);
    for (size_t i0 = 0; i0 < ready.size(); i0 += kMultiMaxTensors) {
      const size_t i1 = std::min(ready.size(), i0 + kMultiMaxTensors);
      if (i1 - i0 < 2) break;  // a single filter keeps its own channels_last node
      std::vector<ir::Value*> ins;
      std::vector<ir::TensorType> types;
      for (size_t i = i0; i < i1; ++i) {
        ins.push_back(map.at(ready[i]));
        types.push_back(channels_last_type(ready[i]));
      }
      Result<ir::Node*> n = out.create_node(std::string(kChannelsLastMultiOp), std::move(ins), std::move(types));
      if (!n.is_ok()) return n.status();
      for (size_t i = i0; i < i1; ++i) batched_out[ready[i]] = n.value()->output(static_cast<int32_t>(i - i0));
    }
    return Status::ok();
  };

  // graph-input filters of the lowered input gradients, in first-use order, each once: all of them are defined
  // before the first input gradient, where one launch flips them all (fh_conv_filter_flip_multi)
  std::vector<const ir::Value*> flip_batched;
  {
    std::unordered_set<const ir::Value*> seen;
    for (const ir::Node* n : src.topological_order()) {
      if (!plan_grad_input(n).ok) continue;
      const ir::Value* w = n->inputs()[1];
      if (w->producer() == nullptr || w->producer()->op() != ir::kGraphInputOp || seen.count(w)) continue;
      if (w->type().shape.dim(2) * w->type().shape.dim(3) > FH_FLIP_MAX_TAPS) continue;
      seen.insert(w);
      flip_batched.push_back(w);
    }
  }
  std::unordered_map<const ir::Value*, ir::Value*> flip_out;  // source filter -> its flipped value
  bool flips_emitted = false;
  auto emit_flips = [&]() -> Status {
    flips_emitted = true;
    for (size_t i0 = 0; i0 < flip_batched.size(); i0 += FH_FLIP_MAX) {
      const size_t i1 = std::min(flip_batched.size(), i0 + size_t{FH_FLIP_MAX});
      if (i1 - i0 < 2) break;  // a single filter keeps its own flip node
      std::vector<ir::Value*> ins;
      std::vector<ir::TensorType> types;
      for (size_t i = i0; i < i1; ++i) {
        ins.push_back(map.at(flip_batched[i]));
        ir::TensorType t = flip_batched[i]->type();
        const Shape& ws = t.shape;
        t.shape = Shape({ws.dim(1), ws.dim(2), ws.dim(3), ws.dim(0)});
        types.push_back(t);
      }
      Result<ir::Node*> n = out.create_node(std::string(kFilterFlipMultiOp), std::move(ins), std::move(types));
      if (!n.is_ok()) return n.status();
      for (size_t i = i0; i < i1; ++i) flip_out[flip_batched[i]] = n.value()->output(static_cast<int32_t>(i - i0));
    }
    return Status::ok();
  };

  // Graph inputs first (same order, so the same signature; they have no operands, so the order stays
  // topological): every filter is defined before the first conv, where the batched transpose goes.
  for (const ir::Node* n : src.topological_order()) {
    if (n->op() != ir::kGraphInputOp) continue;
    Result<ir::Value*> v = out.add_graph_input(n->outputs()[0].type());
    if (!v.is_ok()) return v.status();
    map[&n->outputs()[0]] = v.value();
  }
  for (const ir::Node* n : src.topological_order()) {
    if (n->op() == ir::kGraphInputOp) continue;
    std::vector<ir::Value*> ins;
    for (const ir::Value* in : n->inputs()) ins.push_back(map.at(in));
    if (const GradInputLowering gi = plan_grad_input(n); gi.ok) {
      ir::TensorType wt = ins[1]->type(), dt = ins[0]->type();
      wt.shape = Shape({gi.cin, gi.kh, gi.kw, gi.cout});
      if (!flips_emitted) FRAME_RETURN_IF_ERROR(emit_flips());
      ir::Value* flipped = nullptr;
      if (auto it = flip_out.find(n->inputs()[1]); it != flip_out.end()) {
        flipped = it->second;
      } else {
        Result<ir::Node*> flip = out.create_node(std::string(kFilterFlipOp), {ins[1]}, {wt});
        if (!flip.is_ok()) return flip.status();
        flipped = flip.value()->output(0);
      }
      ir::Value* dy_cl = nullptr;
      const bool dy_nhwc = nhwc.count(n->inputs()[0]) != 0;
      if (gi.sh == 1 && gi.sw == 1) {
        if (dy_nhwc) {
          dy_cl = ins[0];
        } else {
          Result<ir::Value*> v = channels_last(ins[0]);
          if (!v.is_ok()) return v.status();
          dy_cl = v.value();
        }
      } else {
        dt.shape = Shape({gi.n, gi.hu, gi.wu, gi.cout});
        Result<ir::Node*> d = out.create_node(std::string(kDilateNhwcOp), {ins[0]}, {dt});
        if (!d.is_ok()) return d.status();
        d.value()->set_attr("stride", ir::AttrValue{std::vector<int64_t>{gi.sh, gi.sw}});
        if (dy_nhwc) d.value()->set_attr("in_nhwc", ir::AttrValue{int64_t{1}});
        dy_cl = d.value()->output(0);
      }
      Result<ir::Node*> c =
          out.create_node(std::string(kConvNhwcOp), {dy_cl, flipped}, {lowered_type(&n->outputs()[0])});
      if (!c.is_ok()) return c.status();
      if (nhwc.count(&n->outputs()[0])) c.value()->set_attr("out_nhwc", ir::AttrValue{int64_t{1}});
      c.value()->set_attr("stride", ir::AttrValue{std::vector<int64_t>{1, 1}});
      c.value()->set_attr("padding", ir::AttrValue{std::vector<int64_t>{gi.kh - 1 - gi.ph, gi.kw - 1 - gi.pw}});
      c.value()->set_attr("groups", ir::AttrValue{int64_t{1}});
      c.value()->set_attr("n_main_inputs", ir::AttrValue{int64_t{2}});
      c.value()->set_attr("filter_hw", ir::AttrValue{std::vector<int64_t>{gi.kh, gi.kw}});
      map[&n->outputs()[0]] = c.value()->output(0);
      continue;
    }
    if (const GradFilterLowering gf = plan_grad_filter(n); gf.ok) {
      ir::Value* x_cl = nullptr;
      if (gf.c8) {
        Result<ir::Value*> px = pack_c8(ins[0]);
        if (!px.is_ok()) return px.status();
        x_cl = px.value();
      } else if (nhwc.count(n->inputs()[0])) {
        x_cl = ins[0];
      } else {
        Result<ir::Value*> v = channels_last(ins[0]);
        if (!v.is_ok()) return v.status();
        x_cl = v.value();
      }
      Result<ir::Value*> dy_cl = nhwc.count(n->inputs()[1]) ? Result<ir::Value*>(ins[1]) : channels_last(ins[1]);
      if (!dy_cl.is_ok()) return dy_cl.status();
      ir::TensorType wst = n->outputs()[0].type();
      wst.dtype = DType::of<float>();
      wst.shape = Shape({gf.workspace / 4});
      Result<ir::Node*> c = out.create_node(std::string(kConvWgradOp), {x_cl, dy_cl.value()}, {n->outputs()[0].type(), wst});
      if (!c.is_ok()) return c.status();
      for (const auto& [k, v] : n->attrs()) c.value()->set_attr(k, v);
      map[&n->outputs()[0]] = c.value()->output(0);
      continue;
    }
    const ConvLowering p = plan_conv(n);
    if (p.ok) {
      const int64_t* geom = p.geom;
      ir::Value* x_cl = nullptr;
      ir::Value* w_cl = nullptr;
      bool in_nchw = false, w_oihw = false;
      if (p.c8) {
        ir::TensorType tw = ins[1]->type();
        tw.shape = Shape({geom[4], fh_conv_c8_filter_k(geom[5], geom[6])});
        Result<ir::Value*> px = pack_c8(ins[0]);
        if (!px.is_ok()) return px.status();
        Result<ir::Node*> pw = out.create_node(std::string(kPackFilterC8Op), {ins[1]}, {tw});
        if (!pw.is_ok()) return pw.status();
        x_cl = px.value();
        w_cl = pw.value()->output(0);
      } else {
        if (!batched_emitted) FRAME_RETURN_IF_ERROR(emit_batched());
        if (nhwc.count(n->inputs()[0])) {
          x_cl = ins[0];  // already channels-last
        } else if (reads_nchw(n, p)) {
          x_cl = ins[0];  // NCHW, read by the resident-patch kernel itself (FH_CONV_IN_NCHW)
          in_nchw = true;
          w_oihw = takes_oihw(n, p);
        } else {
          Result<ir::Value*> xv = channels_last(ins[0]);
          if (!xv.is_ok()) return xv.status();
          x_cl = xv.value();
        }
        if (w_oihw) {
          w_cl = ins[1];  // [Cout][Cin][KH][KW], transposed by the band kernel on its way into LDS
        } else if (auto it = batched_out.find(n->inputs()[1]); it != batched_out.end()) {
          w_cl = it->second;
        } else {
          Result<ir::Value*> wv = channels_last(ins[1]);
          if (!wv.is_ok()) return wv.status();
          w_cl = wv.value();
        }
      }
      std::vector<ir::Value*> conv_ins = ins;
      conv_ins[0] = x_cl;
      conv_ins[1] = w_cl;
      std::vector<ir::TensorType> conv_outs{lowered_type(&n->outputs()[0])};
      if (!p.c8 && !in_nchw && nhwc.count(&n->outputs()[0])) {
        // split K (fh_conv2d_nhwc_fwd_split): its fp32 partials as a second, planned output
        int32_t splits = 0;
        const int64_t ws = fh_conv2d_nhwc_split_workspace(conv_dtype_code(n->inputs()[0]->type()), geom, FH_CONV_OUT_NHWC, &splits);
        if (ws > 0) {
          ir::TensorType wst = conv_outs[0];
          wst.dtype = DType::of<float>();
          wst.shape = Shape({ws / 4});
          conv_outs.push_back(wst);
        }
      }
      Result<ir::Node*> c = out.create_node(std::string(kConvNhwcOp), std::move(conv_ins), std::move(conv_outs));
      if (!c.is_ok()) return c.status();
      for (const auto& [k, v] : n->attrs()) c.value()->set_attr(k, v);
      if (nhwc.count(&n->outputs()[0])) c.value()->set_attr("out_nhwc", ir::AttrValue{int64_t{1}});
      if (in_nchw) c.value()->set_attr("in_nchw", ir::AttrValue{int64_t{1}});
      if (w_oihw) c.value()->set_attr("w_oihw", ir::AttrValue{int64_t{1}});
      if (n->op() == "conv2d") c.value()->set_attr("n_main_inputs", ir::AttrValue{static_cast<int64_t>(ins.size())});
      c.value()->set_attr("filter_hw", ir::AttrValue{std::vector<int64_t>{geom[5], geom[6]}});
      map[&n->outputs()[0]] = c.value()->output(0);
      continue;
    }
    if (auto it = folded_reshape.find(n); it != folded_reshape.end()) {  // the pool below already has its type
      map[&n->outputs()[0]] = map.at(n->inputs()[0]);
      continue;
    }
    std::vector<ir::TensorType> types;
    for (const ir::Value& o : n->outputs()) types.push_back(lowered_type(&o));
    if (auto it = reshaped_pool.find(n); it != reshaped_pool.end()) types[0] = it->second->outputs()[0].type();
    std::string op(n->op());
    if (n->outputs().size() == 1 && nhwc.count(&n->outputs()[0])) {  // pools of channels-last activations
      if (op == "max_pool2d") op = std::string(kMaxPoolNhwcOp);
      if (op == "avg_pool2d") op = std::string(kAvgPoolNhwcOp);
      if (op == "avg_pool2d_grad_internal") op = std::string(kAvgPoolGradNhwcOp);
    }
    const bool sum_nhwc = op == "sum" && nhwc.count(n->inputs()[0]);
    if (op == "sum") {
      // every axis but the last of the (lowered) input reduced: the two-pass column sum
      const Shape& xs = ins[0]->type().shape;
      const auto* ax = attr_of<std::vector<int64_t>>(n, "axes");
      const auto* kd = attr_of<bool>(n, "keepdims");
      std::vector<int64_t> axes = sum_nhwc ? *nhwc_sum_axes(n) : (ax ? *ax : std::vector<int64_t>{});
      bool rows_form = ax != nullptr && !(kd && *kd) && xs.rank() >= 2 && static_cast<int64_t>(axes.size()) == xs.rank() - 1;
      for (size_t i = 0; rows_form && i < axes.size(); ++i) rows_form = axes[i] == static_cast<int64_t>(i);
      const ir::TensorType& xt = ins[0]->type();
      const int32_t dt = xt.dtype.code() == DTypeCode::kBFloat16  ? FH_BF16
                         : xt.dtype.code() == DTypeCode::kFloat16 ? FH_F16
                         : xt.dtype.code() == DTypeCode::kFloat32 ? FH_F32
                                                                  : -1;
      const int64_t cols = rows_form ? xs.dim(xs.rank() - 1) : 0;
      const int64_t ws = rows_form && dt >= 0 ? fh_sum_rows_workspace(dt, xs.numel() / std::max<int64_t>(cols, 1), cols) : -1;
      if (ws > 0 && xs.numel() / cols >= 256) {
        ir::TensorType wst = types[0];
        wst.dtype = DType::of<float>();
        wst.shape = Shape({ws / 4});
        Result<ir::Node*> c = out.create_node(std::string(kSumRowsOp), std::move(ins), {types[0], wst});
        if (!c.is_ok()) return c.status();
        map[&n->outputs()[0]] = c.value()->output(0);
        continue;
      }
    }
    Result<ir::Node*> c = out.create_node(op, std::move(ins), std::move(types));
    if (!c.is_ok()) return c.status();
    for (const auto& [k, v] : n->attrs()) c.value()->set_attr(k, v);
    if (sum_nhwc) c.value()->set_attr("axes", ir::AttrValue{*nhwc_sum_axes(n)});
    if (op == "reshape" && nhwc.count(&n->outputs()[0]))  // [N,C,1,1] kept as [N,1,1,C]: same bytes
      c.value()->set_attr("target_shape", ir::AttrValue{lowered_type(&n->outputs()[0]).shape});
    for (size_t i = 0; i < n->outputs().size(); ++i) map[&n->outputs()[i]] = c.value()->output(static_cast<int32_t>(i));
  }
  for (const ir::Value* o : src.outputs()) FRAME_RETURN_IF_ERROR(out.mark_output(map.at(o)));
  return out;
}

// ---- attention ---------------------------------------------------------------------------------------------

const ir::Node* producer_op(const ir::Value* v, std::string_view op, size_t n_inputs) {
  const ir::Node* p = v->producer();
  return p != nullptr && p->op() == op && p->inputs().size() == n_inputs && p->outputs().size() == 1 ? p : nullptr;
}

// x when v = slice(x) {axis, start, stop} with exactly these attributes, else nullptr.
const ir::Node* slice_of(const ir::Value* v, int64_t axis, int64_t start, int64_t stop) {
  const ir::Node* s = producer_op(v, "slice", 1);
  if (s == nullptr) return nullptr;
  const int64_t* a = attr_of<int64_t>(s, "axis");
  const int64_t* b = attr_of<int64_t>(s, "start");
  const int64_t* e = attr_of<int64_t>(s, "stop");
  return a && b && e && *a == axis && *b == start && *e == stop ? s : nullptr;
}

// Value of a constant node whose payload is one repeated number, narrowed to `dtype` the way
// fill_tensor_from_constant_attrs narrows it (double -> float -> dtype, round to nearest even).
std::optional<float> splat_value(const ir::Node* c, DType dtype) {
  if (c == nullptr || c->op() != ops::kConstantOpName || !c->inputs().empty()) return std::nullopt;
  const auto* vals = attr_of<std::vector<double>>(c, "value");
  if (vals == nullptr || vals->empty()) return std::nullopt;
  for (double x : *vals)
    if (!(x == vals->front())) return std::nullopt;
  const float f = static_cast<float>(vals->front());
  if (dtype.code() == DTypeCode::kBFloat16) return bfloat16_to_float(float_to_bfloat16(f));
  if (dtype.code() == DTypeCode::kFloat16) return float16_to_float(float_to_float16(f));
  return std::nullopt;
}

struct AttentionMatch {
  ir::Value* q = nullptr;
  ir::Value* k = nullptr;
  ir::Value* v = nullptr;
  int64_t batch = 0, seq = 0, heads = 0, dh = 0;
  float scale = 0.0f;
  std::vector<const ir::Node*> absorbed;  // every node of the decomposition, the batch concat included
};

// Matches the decomposition the reference's MultiHeadAttention emits (reference: src/nn/layers.cpp:1014-1080),
// rooted at the batch concat `root`:
//   root = concat_axis0_b( concat_axis1_h( matmul(softmax(mul(matmul(Qbh, transpose(Kbh, [1,0])), C)), Vbh) ) )
//   Xbh  = slice_axis1[h*dh, (h+1)*dh)( slice_axis0[b*seq, (b+1)*seq)(X) )   for X in Q, K, V
// with C a constant splat (either mul operand) and Q, K, V of shape [batch*seq, heads*dh].
std::optional<AttentionMatch> match_attention(const ir::Node* root) {
  if (root->op() != "concat" || root->outputs().size() != 1 || root->inputs().empty()) return std::nullopt;
  const int64_t* axis0 = attr_of<int64_t>(root, "axis");
  const ir::TensorType& ot = root->outputs()[0].type();
  if (axis0 == nullptr || *axis0 != 0 || ot.shape.rank() != 2) return std::nullopt;
  const int32_t dt = ot.dtype.code() == DTypeCode::kBFloat16 ? FH_BF16 : ot.dtype.code() == DTypeCode::kFloat16 ? FH_F16 : -1;
  if (dt < 0) return std::nullopt;
  AttentionMatch m;
  m.batch = static_cast<int64_t>(root->inputs().size());
  const ir::Node* c1 = root->inputs()[0]->producer();
  if (c1 == nullptr || c1->op() != "concat" || c1->inputs().empty()) return std::nullopt;
  m.heads = static_cast<int64_t>(c1->inputs().size());
  const Shape& head_shape = c1->inputs()[0]->type().shape;
  if (head_shape.rank() != 2) return std::nullopt;
  m.seq = head_shape.dim(0);
  m.dh = head_shape.dim(1);
  if (ot.shape != Shape({m.batch * m.seq, m.heads * m.dh}) || fh_attention_supported(dt, m.seq, m.dh) != 1)
    return std::nullopt;
  std::optional<float> scale;
  m.absorbed.push_back(root);
  for (int64_t b = 0; b < m.batch; ++b) {
    const ir::Value* ob = root->inputs()[static_cast<size_t>(b)];
    const ir::Node* cb = producer_op(ob, "concat", static_cast<size_t>(m.heads));
    if (cb == nullptr || attr_of<int64_t>(cb, "axis") == nullptr || *attr_of<int64_t>(cb, "axis") != 1) return std::nullopt;
    m.absorbed.push_back(cb);
    const int64_t r0 = b * m.seq, r1 = r0 + m.seq;
    // the row slices of Q, K, V for this batch (shared by its heads)
    const ir::Node* rows[3] = {nullptr, nullptr, nullptr};
    for (int64_t h = 0; h < m.heads; ++h) {
      const int64_t c0 = h * m.dh, c1h = c0 + m.dh;
      const ir::Node* pv = producer_op(cb->inputs()[static_cast<size_t>(h)], "matmul", 2);
      if (pv == nullptr) return std::nullopt;
      const ir::Node* sm = producer_op(pv->inputs()[0], "softmax", 1);
      if (sm == nullptr) return std::nullopt;
      const ir::Node* mul = producer_op(sm->inputs()[0], "mul", 2);
      if (mul == nullptr) return std::nullopt;
      const ir::Value* s = mul->inputs()[0];
      std::optional<float> sc = splat_value(mul->inputs()[1]->producer(), ot.dtype);
      if (!sc) {
        s = mul->inputs()[1];
        sc = splat_value(mul->inputs()[0]->producer(), ot.dtype);
      }
      if (!sc || (scale && *scale != *sc)) return std::nullopt;
      scale = sc;
      const ir::Node* qk = producer_op(s, "matmul", 2);
      if (qk == nullptr) return std::nullopt;
      const ir::Node* kt = producer_op(qk->inputs()[1], "transpose", 1);
      const auto* perm = kt ? attr_of<std::vector<int64_t>>(kt, "perm") : nullptr;
      if (perm == nullptr || *perm != std::vector<int64_t>{1, 0}) return std::nullopt;
      const ir::Value* heads_in[3] = {qk->inputs()[0], kt->inputs()[0], pv->inputs()[1]};
      for (int i = 0; i < 3; ++i) {
        const ir::Node* col = slice_of(heads_in[i], 1, c0, c1h);
        if (col == nullptr) return std::nullopt;
        const ir::Node* row = slice_of(col->inputs()[0], 0, r0, r1);
        if (row == nullptr || (rows[i] != nullptr && rows[i] != row)) return std::nullopt;
        ir::Value* x = row->inputs()[0];
        ir::Value*& want = i == 0 ? m.q : i == 1 ? m.k : m.v;
        if (want != nullptr && want != x) return std::nullopt;
        want = x;
        if (rows[i] == nullptr) m.absorbed.push_back(row);
        rows[i] = row;
        m.absorbed.push_back(col);
      }
      m.absorbed.insert(m.absorbed.end(), {pv, sm, mul, qk, kt});
    }
  }
  for (const ir::Value* x : {m.q, m.k, m.v})
    if (x->type().shape != ot.shape || !(x->type().dtype == ot.dtype)) return std::nullopt;
  m.scale = *scale;
  return m;
}

// Replaces every matched attention decomposition by one kAttentionOp node. Nodes of a decomposition whose
// results are also used outside it (or are graph outputs) keep the decomposition as it is. The graph is rebuilt in
// topological order without the nodes the rewrite leaves unused (the shared scale constant among them).
Status lower_attention(ir::Graph& g) {
  std::unordered_map<const ir::Value*, std::vector<const ir::Node*>> users;
  for (const ir::Node* n : g.topological_order())
    for (const ir::Value* v : n->inputs()) users[v].push_back(n);
  std::unordered_set<const ir::Value*> graph_outputs(g.outputs().begin(), g.outputs().end());

  std::unordered_map<const ir::Node*, AttentionMatch> roots;
  std::unordered_set<const ir::Node*> absorbed;
  for (const ir::Node* n : g.topological_order()) {
    std::optional<AttentionMatch> m = match_attention(n);
    if (!m) continue;
    const std::unordered_set<const ir::Node*> mine(m->absorbed.begin(), m->absorbed.end());
    bool closed = true;
    for (const ir::Node* a : m->absorbed) {
      if (absorbed.count(a)) closed = false;
      if (a == n) continue;
      for (const ir::Value& o : a->outputs()) {
        if (graph_outputs.count(&o)) closed = false;
        for (const ir::Node* u : users[&o])
          if (!mine.count(u)) closed = false;
      }
    }
    if (!closed) continue;
    absorbed.insert(m->absorbed.begin(), m->absorbed.end());
    roots.emplace(n, std::move(*m));
  }
  if (roots.empty()) return Status::ok();

  // Liveness after the rewrite: a matched root reads q, k, v instead of its own inputs.
  const std::vector<ir::Node*> order = g.topological_order();
  std::unordered_set<const ir::Node*> live;
  for (const ir::Value* o : g.outputs())
    if (o->producer()) live.insert(o->producer());
  for (auto it = order.rbegin(); it != order.rend(); ++it) {
    const ir::Node* n = *it;
    if (!live.count(n)) continue;
    if (auto r = roots.find(n); r != roots.end()) {
      for (const ir::Value* x : {r->second.q, r->second.k, r->second.v})
        if (x->producer()) live.insert(x->producer());
      continue;
    }
    for (const ir::Value* x : n->inputs())
      if (x->producer()) live.insert(x->producer());
  }

  std::unordered_map<const ir::Value*, ir::Value*> map;
  ir::Graph out{std::string(g.name())};
  for (const ir::Node* n : order) {
    if (n->op() == ir::kGraphInputOp) {
      Result<ir::Value*> v = out.add_graph_input(n->outputs()[0].type());
      if (!v.is_ok()) return v.status();
      map[&n->outputs()[0]] = v.value();
      continue;
    }
    if (!live.count(n)) continue;
    if (auto r = roots.find(n); r != roots.end()) {
      const AttentionMatch& m = r->second;
      Result<ir::Node*> a = out.create_node(std::string(kAttentionOp), {map.at(m.q), map.at(m.k), map.at(m.v)},
                                            {n->outputs()[0].type()});
      if (!a.is_ok()) return a.status();
      a.value()->set_attr("batch", ir::AttrValue{m.batch});
      a.value()->set_attr("seq", ir::AttrValue{m.seq});
      a.value()->set_attr("heads", ir::AttrValue{m.heads});
      a.value()->set_attr("dh", ir::AttrValue{m.dh});
      a.value()->set_attr("scale", ir::AttrValue{static_cast<double>(m.scale)});
      map[&n->outputs()[0]] = a.value()->output(0);
      continue;
    }
    std::vector<ir::Value*> ins;
    for (const ir::Value* in : n->inputs()) ins.push_back(map.at(in));
    std::vector<ir::TensorType> types;
    for (const ir::Value& o : n->outputs()) types.push_back(o.type());
    Result<ir::Node*> c = out.create_node(std::string(n->op()), std::move(ins), std::move(types));
    if (!c.is_ok()) return c.status();
    for (const auto& [k, v] : n->attrs()) c.value()->set_attr(k, v);
    for (size_t i = 0; i < n->outputs().size(); ++i) map[&n->outputs()[i]] = c.value()->output(static_cast<int32_t>(i));
  }
  for (const ir::Value* o : g.outputs()) FRAME_RETURN_IF_ERROR(out.mark_output(map.at(o)));
  g = std::move(out);
  return Status::ok();
}

class HipExecutable final : public hal::Executable {
 public:
  HipExecutable(ops::ExecutablePlan plan, HipAllocator& alloc, Device device, hal::CompileOptions options)
      : plan_(std::move(plan)), alloc_(&alloc), device_(device), options_(std::move(options)) {
    for (const auto& t : plan_.input_types) in_sig_.push_back({t.dtype, t.shape});
    for (const auto& t : plan_.output_types) out_sig_.push_back({t.dtype, t.shape});
  }

  Status materialize_constants() {
    for (size_t i = 0; i < plan_.steps.size(); ++i) {
      const ops::ExecutablePlanStep& s = plan_.steps[i];
      if (s.op != ops::kConstantOpName) continue;
      const ir::TensorType& t = s.output_types[0];
      const size_t bytes = static_cast<size_t>(t.shape.numel()) * t.dtype.itemsize();
      std::vector<unsigned char> host(std::max<size_t>(bytes, 1));
      Result<Tensor> dev = Tensor::empty(t.shape, t.dtype, device_, *alloc_);
      if (!dev.is_ok()) return dev.status();
      // fill_tensor_from_constant_attrs writes through raw_data(); give it a host tensor over `host`.
      struct HostAlloc final : hal::Allocator {
        void* p;
        explicit HostAlloc(void* q) : p(q) {}
        Result<void*> allocate(size_t, size_t) override { return p; }
        void deallocate(void*) override {}
      } ha(host.data());
      Result<Tensor> h = Tensor::empty(t.shape, t.dtype, cpu_device(), ha);
      if (!h.is_ok()) return h.status();
      FRAME_RETURN_IF_ERROR(ops::fill_tensor_from_constant_attrs(s.attrs, h.value()));
      if (bytes > 0)
        FRAME_HIP_RETURN_IF_ERROR(fh_memcpy(dev.value().raw_data(), host.data(), bytes, FH_H2D, nullptr),
                                  "HipExecutable: constant upload");
      constants_.emplace(i, dev.value());
    }
    return Status::ok();
  }

  Status run(std::span<const Tensor> inputs, std::span<Tensor> outputs, hal::Stream& stream) override {
    FRAME_RETURN_IF_ERROR(hal::validate_io_signature(inputs, in_sig_, "HipExecutable::run: input"));
    FRAME_RETURN_IF_ERROR(hal::validate_io_signature(outputs, out_sig_, "HipExecutable::run: output"));
    FRAME_RETURN_IF_ERROR(hal::validate_tensor_devices(inputs, device_, "HipExecutable::run: input"));
    FRAME_RETURN_IF_ERROR(hal::validate_tensor_devices(outputs, device_, "HipExecutable::run: output"));
    void* sh = stream.native_handle();
    // Per-stream state is keyed by the HipStream's process-unique id (a destroyed stream's handle address can come
    // back for a new stream). A stream of another backend gets no cached state: a transient arena for this run.
    const uint64_t sid = hip_stream_id(stream);
    std::shared_ptr<Storage> arena;
    {
      std::lock_guard<std::mutex> lock(mu_);
      prune_stream_state_locked(sid);
      if (plan_.arena_total_bytes > 0) {
        StreamArena* a = sid != 0 ? &arenas_[sid] : nullptr;
        if (a == nullptr || !a->storage) {
          Result<std::shared_ptr<Storage>> st = Storage::allocate(*alloc_, plan_.arena_total_bytes, kDefaultAlignment, device_);
          if (!st.is_ok()) return st.status();
          if (a != nullptr) a->storage = st.value();
          arena = st.value();
        } else {
          arena = a->storage;
        }
        if (a != nullptr) a->last_use = ++use_clock_;
      }
    }
    // Replay (opt-in, FRAME_HIP_GRAPHS=1): the second run on a stream with the same input and output addresses
    // captures the step sequence into a HIP graph, and later runs with those addresses launch that graph instead
    // of every step; other addresses run the steps directly. Off by default: on this ROCm a graph launch costs
    // ~10 us more than launching its kernels (measured: C1 forward 23.8 -> 29.8 us, a 1024^3 GEMM 7 -> 18.5 us),
    // and every workload here keeps the GPU busy without it.
    if (sh == nullptr || sid == 0 || !graphs_enabled() || any_unaligned(inputs, outputs))
      return run_steps(inputs, outputs, stream, arena);
    std::vector<const void*> key;
    for (const Tensor& t : inputs) key.push_back(t.raw_data());
    for (const Tensor& t : outputs) key.push_back(t.raw_data());
    bool capture = false;
    {
      std::lock_guard<std::mutex> lock(mu_);
      GraphCache& gc = graphs_[sid];
      if (gc.exec != nullptr && gc.key == key) {
        FRAME_HIP_RETURN_IF_ERROR(fh_graph_launch(gc.exec, sh), "HipExecutable: graph replay");
        return Status::ok();
      }
      if (gc.key != key) {
        if (gc.exec != nullptr) (void)fh_graph_destroy(gc.exec);
        gc.exec = nullptr;
        gc.key = key;
      } else {
        capture = !gc.failed;
      }
    }
    if (!capture) return run_steps(inputs, outputs, stream, arena);
    FRAME_HIP_RETURN_IF_ERROR(fh_graph_begin_capture(sh), "HipExecutable: graph capture");
    const Status st = run_steps(inputs, outputs, stream, arena);
    void* exec = nullptr;
    const fh_status end = fh_graph_end_capture(sh, st.is_ok() ? 1 : 0, &exec);
    std::lock_guard<std::mutex> lock(mu_);
    GraphCache& gc = graphs_[sid];
    if (!st.is_ok() || end != FH_OK || exec == nullptr) {
      gc.failed = true;  // something in the steps cannot be captured: this executable runs them directly
      if (!st.is_ok()) return st;
      return run_steps(inputs, outputs, stream, arena);
    }
    gc.exec = exec;
    FRAME_HIP_RETURN_IF_ERROR(fh_graph_launch(exec, sh), "HipExecutable: graph replay");
    return Status::ok();
  }

  // Test hook: a run on a transient arena, eager, with the given step outputs copied to host memory as they are
  // produced.
  Status run_tapped(std::span<const Tensor> inputs, std::span<Tensor> outputs, hal::Stream& stream,
                    std::span<const HipStepTap> taps) {
    FRAME_RETURN_IF_ERROR(hal::validate_io_signature(inputs, in_sig_, "HipExecutable::run: input"));
    FRAME_RETURN_IF_ERROR(hal::validate_io_signature(outputs, out_sig_, "HipExecutable::run: output"));
    FRAME_RETURN_IF_ERROR(hal::validate_tensor_devices(inputs, device_, "HipExecutable::run: input"));
    FRAME_RETURN_IF_ERROR(hal::validate_tensor_devices(outputs, device_, "HipExecutable::run: output"));
    std::shared_ptr<Storage> arena;
    if (plan_.arena_total_bytes > 0) {
      Result<std::shared_ptr<Storage>> st = Storage::allocate(*alloc_, plan_.arena_total_bytes, kDefaultAlignment, device_);
      if (!st.is_ok()) return st.status();
      arena = st.value();
    }
    FRAME_RETURN_IF_ERROR(run_steps(inputs, outputs, stream, arena, taps));
    FRAME_HIP_RETURN_IF_ERROR(fh_stream_synchronize(stream.native_handle()), "step tap: final drain");
    return Status::ok();
  }

  // One line per plan step: "index op" (the lowered graph's non-input nodes in order).
  std::string step_list() const {
    std::string out;
    for (size_t i = 0; i < plan_.steps.size(); ++i) out += std::to_string(i) + " " + plan_.steps[i].op + "\n";
    return out;
  }

  ~HipExecutable() override {
    for (auto& [s, gc] : graphs_)
      if (gc.exec != nullptr) (void)fh_graph_destroy(gc.exec);
  }

 private:
  // Drops the arenas and graphs of destroyed streams (their memory returns to the allocator, which reuses it only
  // once the device is idle), and keeps at most kMaxStreamArenas arenas, evicting the least recently used, so an
  // executable run on ever new streams (run_with_allocated_outputs creates one per call) holds bounded memory.
  void prune_stream_state_locked(uint64_t current) {
    for (auto it = arenas_.begin(); it != arenas_.end();)
      it = (it->first != current && !hip_stream_alive(it->first)) ? arenas_.erase(it) : std::next(it);
    for (auto it = graphs_.begin(); it != graphs_.end();) {
      if (it->first != current && !hip_stream_alive(it->first)) {
        if (it->second.exec != nullptr) (void)fh_graph_destroy(it->second.exec);
        it = graphs_.erase(it);
      } else {
        ++it;
      }
    }
    while (arenas_.size() > kMaxStreamArenas) {
      auto lru = arenas_.end();
      for (auto it = arenas_.begin(); it != arenas_.end(); ++it)
        if (it->first != current && (lru == arenas_.end() || it->second.last_use < lru->second.last_use)) lru = it;
      if (lru == arenas_.end()) break;
      arenas_.erase(lru);
    }
  }

 public:
  size_t cached_arena_count() {
    std::lock_guard<std::mutex> lock(mu_);
    return arenas_.size();
  }

 private:
  static bool graphs_enabled() {
    const char* v = std::getenv("FRAME_HIP_GRAPHS");
    return v != nullptr && v[0] == '1';
  }

  // The kernels read and write 16-byte vectors where their operands allow it and some (the band conv with its
  // filter kept in the graph's layout) require it. Arena slices and allocator blocks are aligned; a caller's
  // tensor that is a view at an odd offset is not.
  static bool unaligned(const Tensor& t) {
    return t.numel() > 0 && (reinterpret_cast<uintptr_t>(t.raw_data()) & 15) != 0;
  }
  static bool any_unaligned(std::span<const Tensor> inputs, std::span<Tensor> outputs) {
    for (const Tensor& t : inputs)
      if (unaligned(t)) return true;
    for (const Tensor& t : outputs)
      if (unaligned(t)) return true;
    return false;
  }

  Status run_steps(std::span<const Tensor> inputs, std::span<Tensor> outputs, hal::Stream& stream,
                   const std::shared_ptr<Storage>& arena, std::span<const HipStepTap> taps = {}) {
    void* sh = stream.native_handle();
    // After step si: the tapped outputs go to host memory (the stream is drained first, since the arena
    // slice may be reused by a later step).
    auto tap = [&](size_t si, std::span<const Tensor> produced) -> Status {
      for (const HipStepTap& t : taps) {
        if (t.step != si) continue;
        if (t.output >= produced.size()) return Status::make(ErrorCode::kInvalidArgument, "step tap: output index out of range");
        const Tensor& o = produced[t.output];
        const size_t bytes = static_cast<size_t>(o.numel()) * o.dtype().itemsize();
        if (bytes != t.bytes)
          return Status::make(ErrorCode::kInvalidArgument, "step tap: step " + std::to_string(si) + " output holds " +
                                                               std::to_string(bytes) + " bytes, not " + std::to_string(t.bytes));
        FRAME_HIP_RETURN_IF_ERROR(fh_stream_synchronize(sh), "step tap: drain");
        if (bytes > 0) FRAME_HIP_RETURN_IF_ERROR(fh_memcpy(t.host, o.raw_data(), bytes, FH_D2H, nullptr), "step tap: copy");
      }
      return Status::ok();
    };
    std::vector<Tensor> slots(static_cast<size_t>(plan_.slot_count));
    for (size_t i = 0; i < inputs.size(); ++i) {
      slots[i] = inputs[i];
      if (!unaligned(inputs[i])) continue;
      // an input at an unaligned address is copied (stream-ordered) to an aligned block first
      Result<Tensor> e = Tensor::empty(inputs[i].shape(), inputs[i].dtype(), device_, *alloc_);
      if (!e.is_ok()) return e.status();
      const size_t bytes = static_cast<size_t>(inputs[i].numel()) * inputs[i].dtype().itemsize();
      FRAME_HIP_RETURN_IF_ERROR(fh_memcpy(e.value().raw_data(), inputs[i].raw_data(), bytes, FH_D2D, sh),
                                "HipExecutable: unaligned input copy");
      slots[i] = e.value();
    }
    // A slot that is a graph output is produced directly in the first caller tensor naming it, if that tensor is
    // 16-byte aligned; otherwise in a block of its own, copied out at the end like a passed-through input.
    std::unordered_map<int32_t, size_t> direct;
    for (size_t i = 0; i < plan_.output_slots.size(); ++i)
      if (!unaligned(outputs[i])) direct.try_emplace(plan_.output_slots[i], i);

    std::vector<Tensor> step_in, step_out;
    for (size_t si = 0; si < plan_.steps.size(); ++si) {
      const ops::ExecutablePlanStep& s = plan_.steps[si];
      if (auto c = constants_.find(si); c != constants_.end()) {
        const int32_t slot = s.output_slots[0];
        auto d = direct.find(slot);
        if (d == direct.end()) {
          slots[static_cast<size_t>(slot)] = c->second;
        } else {
          Tensor& dst = outputs[d->second];
          const size_t bytes = static_cast<size_t>(dst.numel()) * dst.dtype().itemsize();
          FRAME_HIP_RETURN_IF_ERROR(fh_memcpy(dst.raw_data(), c->second.raw_data(), bytes, FH_D2D, sh),
                                    "HipExecutable: constant output copy");
          slots[static_cast<size_t>(slot)] = dst;
        }
        if (!taps.empty()) FRAME_RETURN_IF_ERROR(tap(si, std::span<const Tensor>(&slots[static_cast<size_t>(slot)], 1)));
        continue;
      }
      step_in.clear();
      step_out.clear();
      for (int32_t slot : s.input_slots) step_in.push_back(slots[static_cast<size_t>(slot)]);
      for (size_t j = 0; j < s.output_types.size(); ++j) {
        const ir::TensorType& t = s.output_types[j];
        auto d = direct.find(s.output_slots[j]);
        if (d != direct.end()) {
          step_out.push_back(outputs[d->second]);
        } else if (s.output_arena_offsets[j].has_value() && t.shape.numel() > 0) {
          step_out.push_back(Tensor::from_storage_slice(arena, *s.output_arena_offsets[j], t.shape, t.dtype, device_));
        } else {
          Result<Tensor> e = Tensor::empty(t.shape, t.dtype, device_, *alloc_);
          if (!e.is_ok()) return e.status();
          step_out.push_back(e.value());
        }
      }
      ops::KernelContext ctx{step_in, step_out, &s.attrs, device_, &stream, &options_};
      Status st = s.kernel(ctx);
      if (!st.is_ok())
        return Status::make(st.code(), "HipExecutable::run: op '" + s.op + "' kernel failed: " + std::string(st.message()));
      for (size_t j = 0; j < s.output_slots.size(); ++j) slots[static_cast<size_t>(s.output_slots[j])] = step_out[j];
      if (!taps.empty()) FRAME_RETURN_IF_ERROR(tap(si, step_out));
    }
    // Outputs that were not written in place: graph inputs passed through, or a value listed twice.
    for (size_t i = 0; i < plan_.output_slots.size(); ++i) {
      const Tensor& src = slots[static_cast<size_t>(plan_.output_slots[i])];
      Tensor& dst = outputs[i];
      if (src.raw_data() == dst.raw_data()) continue;
      const size_t bytes = static_cast<size_t>(src.numel()) * src.dtype().itemsize();
      if (bytes > 0)
        FRAME_HIP_RETURN_IF_ERROR(fh_memcpy(dst.raw_data(), src.raw_data(), bytes, FH_D2D, sh),
                                  "HipExecutable: output copy");
    }
    return Status::ok();
  }


 public:
  std::vector<hal::IoSpec> input_signature() const override { return in_sig_; }
  std::vector<hal::IoSpec> output_signature() const override { return out_sig_; }

 private:
  struct GraphCache {
    std::vector<const void*> key;  // input then output addresses of the captured run
    void* exec = nullptr;          // instantiated graph, or null
    bool failed = false;           // capture failed once: run steps directly from now on
  };
  ops::ExecutablePlan plan_;
  HipAllocator* alloc_;
  Device device_;
  hal::CompileOptions options_;
  std::vector<hal::IoSpec> in_sig_, out_sig_;
  std::unordered_map<size_t, Tensor> constants_;  // step index -> device tensor
  struct StreamArena {
    std::shared_ptr<Storage> storage;
    uint64_t last_use = 0;
  };
  static constexpr size_t kMaxStreamArenas = 4;
  std::mutex mu_;
  uint64_t use_clock_ = 0;
  std::unordered_map<uint64_t, StreamArena> arenas_;  // HipStream id -> arena
  std::unordered_map<uint64_t, GraphCache> graphs_;   // HipStream id -> captured step list
};

}  // namespace

// Whether a matmul_grad node's GEMM is large enough for the tiled kernels: the same threshold as fh_gemm's
// dispatch on a 256-CU device (fp32 from 64 tiles of 64 x 64, 16-bit from 16). Smaller ones stay
// matmul_grad_*_internal and run on fh_matmul_grad's sequential kernel, which reads the transposed operand in place.
bool matmul_grad_wants_gemm(const ir::Node* n) {
  const bool lhs = n->op() == "matmul_grad_lhs_internal";
  if (!lhs && n->op() != "matmul_grad_rhs_internal") return false;
  const Shape& p = n->inputs()[0]->type().shape;
  const Shape& q = n->inputs()[1]->type().shape;
  const int64_t M = lhs ? p.dim(0) : p.dim(1), N = lhs ? q.dim(0) : q.dim(1), K = lhs ? p.dim(1) : p.dim(0);
  const int64_t tiles64 = ((M + 63) / 64) * ((N + 63) / 64);
  const bool f32 = n->inputs()[0]->type().dtype.code() == DTypeCode::kFloat32;
  return (f32 ? tiles64 >= 64 : tiles64 >= 16) || K > 16384;
}

// matmul_grad_lhs_internal(gy, b) = gy * b^T and matmul_grad_rhs_internal(a, gy) = a^T * gy, when large, become a
// transpose of the transposed operand plus a plain matmul, so they run on the tiled GEMM kernels with the same
// products and fp32 accumulation as the reference (src/backends/cpu/kernels/matmul.cpp:187-327). Returns a clone
// of the source when no node qualifies.
Result<ir::Graph> lower_matmul_grads(const ir::Graph& src) {
  const auto& order = src.topological_order();
  const bool any = std::any_of(order.begin(), order.end(), matmul_grad_wants_gemm);
  if (!any) return ir::clone_graph(src);
  std::unordered_map<const ir::Value*, ir::Value*> map;
  ir::Graph out{std::string(src.name())};
  for (const ir::Node* n : order) {
    if (n->op() == ir::kGraphInputOp) {
      Result<ir::Value*> v = out.add_graph_input(n->outputs()[0].type());
      if (!v.is_ok()) return v.status();
      map[&n->outputs()[0]] = v.value();
      continue;
    }
    std::vector<ir::Value*> ins;
    for (const ir::Value* in : n->inputs()) ins.push_back(map.at(in));
    if (matmul_grad_wants_gemm(n)) {
      const bool lhs = n->op() == "matmul_grad_lhs_internal";
      ir::Value* t_in = lhs ? ins[1] : ins[0];  // b of gy*b^T, a of a^T*gy
      ir::TensorType tt = t_in->type();
      tt.shape = Shape({tt.shape.dim(1), tt.shape.dim(0)});
      Result<ir::Node*> t = out.create_node("transpose", {t_in}, {tt});
      if (!t.is_ok()) return t.status();
      t.value()->set_attr("perm", ir::AttrValue{std::vector<int64_t>{1, 0}});
      std::vector<ir::Value*> mm_in = lhs ? std::vector<ir::Value*>{ins[0], t.value()->output(0)}
                                          : std::vector<ir::Value*>{t.value()->output(0), ins[1]};
      Result<ir::Node*> mm = out.create_node("matmul", std::move(mm_in), {n->outputs()[0].type()});
      if (!mm.is_ok()) return mm.status();
      map[&n->outputs()[0]] = mm.value()->output(0);
      continue;
    }
    std::vector<ir::TensorType> types;
    for (const ir::Value& o : n->outputs()) types.push_back(o.type());
    Result<ir::Node*> c = out.create_node(std::string(n->op()), std::move(ins), std::move(types));
    if (!c.is_ok()) return c.status();
    for (const auto& [k, v] : n->attrs()) c.value()->set_attr(k, v);
    for (size_t j = 0; j < n->outputs().size(); ++j) map[&n->outputs()[j]] = c.value()->output(static_cast<int32_t>(j));
  }
  for (const ir::Value* o : src.outputs()) FRAME_RETURN_IF_ERROR(out.mark_output(map.at(o)));
  return out;
}

// add(x, mul(constant s, y)) with x and y graph inputs of one shape and dtype (either operand order), the mul used only by that add: the
// SGD update graph's parameter updates (reference: src/compiler/autograd.cpp:418-440). Runs of up to FH_AXPY_MAX
// such pairs of one dtype become one kAxpyMultiOp node (one launch instead of two per parameter); the constant
// goes with them when nothing else reads it. Results are bit-identical: the product is rounded as the mul node
// stores it, then added in the add node's operand order.
Status lower_scaled_adds(ir::Graph& g) {
  std::unordered_map<const ir::Value*, int> uses;
  for (const ir::Node* n : g.topological_order())
    for (const ir::Value* v : n->inputs()) ++uses[v];
  for (const ir::Value* v : g.outputs()) uses[v] += 1000;
  struct Pair {
    ir::Node* add;
    ir::Node* mul;
    ir::Node* c;
    ir::Value* x;
    ir::Value* y;
    float s;
  };
  std::map<int, std::vector<Pair>> by_dtype;
  for (ir::Node* a : g.topological_order()) {
    if (a->op() != "add" || a->inputs().size() != 2 || a->outputs().size() != 1) continue;
    // canonicalize may have swapped the operands of either node; both are commutative in IEEE arithmetic
    auto made_by = [](const ir::Value* v, std::string_view op) { return v->producer() != nullptr && v->producer()->op() == op; };
    const int mi = made_by(a->inputs()[1], "mul") ? 1 : 0;
    ir::Value* x = a->inputs()[1 - mi];
    ir::Value* m = a->inputs()[mi];
    ir::Node* mul = m->producer();
    if (!made_by(x, ir::kGraphInputOp) || !made_by(m, "mul") || mul->inputs().size() != 2 || uses[m] != 1) continue;
    const int ci = made_by(mul->inputs()[0], ops::kConstantOpName) ? 0 : 1;
    ir::Node* c = mul->inputs()[ci]->producer();
    ir::Value* y = mul->inputs()[1 - ci];
    if (!made_by(mul->inputs()[ci], ops::kConstantOpName) || !made_by(y, ir::kGraphInputOp)) continue;
    const ir::TensorType& t = a->outputs()[0].type();
    if (!(x->type().dtype == t.dtype) || !(y->type().dtype == t.dtype) || !(mul->inputs()[ci]->type().dtype == t.dtype) ||
        x->type().shape != t.shape || y->type().shape != t.shape || mul->inputs()[ci]->type().shape != t.shape)
      continue;
    const int dt = t.dtype.code() == DTypeCode::kFloat32 ? FH_F32 : t.dtype.code() == DTypeCode::kBFloat16 ? FH_BF16
                   : t.dtype.code() == DTypeCode::kFloat16 ? FH_F16 : -1;
    if (dt < 0) continue;
    std::optional<float> sv;
    if (dt == FH_F32) {
      const auto* vals = c != nullptr && c->op() == ops::kConstantOpName && c->inputs().empty()
                             ? attr_of<std::vector<double>>(c, "value") : nullptr;
      if (vals != nullptr && !vals->empty() &&
          std::all_of(vals->begin(), vals->end(), [&](double v) { return v == vals->front(); }))
        sv = static_cast<float>(vals->front());
    } else {
      sv = splat_value(c, t.dtype);
    }
    if (!sv) continue;
    by_dtype[dt].push_back({a, mul, c, x, y, *sv});
  }
  for (auto& [dt, pairs] : by_dtype) {
    for (size_t first = 0; first < pairs.size(); first += FH_AXPY_MAX) {
      const size_t last = std::min(pairs.size(), first + FH_AXPY_MAX);
      if (last - first < 2) break;  // a single pair keeps its two nodes
      std::vector<ir::Value*> ins;
      std::vector<ir::TensorType> types;
      std::vector<double> scales;
      for (size_t i = first; i < last; ++i) {
        ins.push_back(pairs[i].x);
        ins.push_back(pairs[i].y);
        types.push_back(pairs[i].add->outputs()[0].type());
        scales.push_back(pairs[i].s);
      }
      Result<ir::Node*> f = g.create_node(std::string(kAxpyMultiOp), std::move(ins), std::move(types));
      if (!f.is_ok()) return f.status();
      f.value()->set_attr("scales", ir::AttrValue{scales});
      for (size_t i = first; i < last; ++i) {
        FRAME_RETURN_IF_ERROR(g.replace_all_uses(pairs[i].add->output(0), f.value()->output(static_cast<int>(i - first))));
        FRAME_RETURN_IF_ERROR(g.erase_node(pairs[i].add));
        FRAME_RETURN_IF_ERROR(g.erase_node(pairs[i].mul));
        if (--uses[pairs[i].c->output(0)] == 0) FRAME_RETURN_IF_ERROR(g.erase_node(pairs[i].c));
      }
    }
  }
  return Status::ok();
}

// A softmax whose input is a fused matmul (any_order) of at most 16 columns, used by nothing else, runs in that
// GEMM's launch: the matmul node gets row_softmax = 1 (fh_gemm_ex with FH_GEMM_ROW_SOFTMAX) and the softmax node
// goes. C1's classifier layer (matmul, bias add, softmax over 10 classes) becomes one kernel.
Status lower_gemm_softmax(ir::Graph& g) {
  std::unordered_map<const ir::Value*, int> uses;
  for (const ir::Node* n : g.topological_order())
    for (const ir::Value* v : n->inputs()) ++uses[v];
  for (const ir::Value* v : g.outputs()) uses[v] += 1000;
  const std::vector<ir::Node*> snapshot = g.topological_order();
  for (ir::Node* sm : snapshot) {
    if (sm->op() != "softmax" || sm->inputs().size() != 1 || sm->outputs().size() != 1) continue;
    ir::Value* v = sm->inputs()[0];
    ir::Node* p = v->producer();
    if (p == nullptr || p->op() != kGemmEpilogueOp || uses[v] != 1) continue;
    const auto* any = attr_of<int64_t>(p, "any_order");
    const auto* n_main = attr_of<int64_t>(p, "n_main_inputs");
    if (any == nullptr || *any == 0 || n_main == nullptr || *n_main != 2) continue;
    const ir::TensorType& ot = p->outputs()[0].type();
    if (ot.shape.rank() != 2 || ot.shape.dim(1) > 16 || ot.shape.dim(0) > 262140) continue;
    const ir::TensorType& st = sm->outputs()[0].type();
    if (!(ot.shape == st.shape) || !(ot.dtype == st.dtype)) continue;
    p->set_attr("row_softmax", ir::AttrValue{int64_t{1}});
    FRAME_RETURN_IF_ERROR(g.replace_all_uses(sm->output(0), p->output(0)));
    FRAME_RETURN_IF_ERROR(g.erase_node(sm));
  }
  return Status::ok();
}

// Matmuls (plain, or epilogue nodes with two main inputs) of a 16-bit dtype that read the same A value, with equal
// B shapes, output types and epilogue programs, merged in groups of up to FH_GEMM_MAX_GROUPS into one
// kGemmGroupedOp node, when every operand of the group is produced before the group's first member (so the
// merged node can take that member's place and no member depends on another).
Status lower_grouped_gemms(ir::Graph& g) {
  struct Member {
    ir::Node* node;
    size_t pos;
  };
  std::unordered_map<const ir::Node*, size_t> pos;
  {
    const auto& order = g.topological_order();
    for (size_t i = 0; i < order.size(); ++i) pos[order[i]] = i;
  }
  auto program = [](const ir::Node* n) -> std::vector<int64_t> {
    const auto* p = attr_of<std::vector<int64_t>>(n, "ep_ops");
    return p != nullptr ? *p : std::vector<int64_t>{};
  };
  std::map<std::string, std::vector<Member>> groups;  // key -> members in topological order
  for (ir::Node* n : g.topological_order()) {
    const bool mm = n->op() == "matmul" && n->inputs().size() == 2;
    const auto* n_main = attr_of<int64_t>(n, "n_main_inputs");
    const bool epi = n->op() == kGemmEpilogueOp && n_main != nullptr && *n_main == 2;
    if ((!mm && !epi) || n->outputs().size() != 1 || attr_of<int64_t>(n, "row_softmax") != nullptr) continue;
    const ir::TensorType& ot = n->outputs()[0].type();
    if (ot.dtype.code() != DTypeCode::kBFloat16 && ot.dtype.code() != DTypeCode::kFloat16) continue;
    const ir::TensorType& bt = n->inputs()[1]->type();
    if (bt.shape.rank() != 2 || ot.shape.rank() != 2) continue;
    std::string key = std::to_string(reinterpret_cast<uintptr_t>(n->inputs()[0])) + "|" + bt.shape.to_string() + "|" +
                      ot.shape.to_string() + "|" + std::to_string(static_cast<int>(ot.dtype.code())) + "|";
    for (int64_t c : program(n)) key += std::to_string(c) + ",";
    groups[key].push_back({n, pos[n]});
  }
  for (auto& [key, members] : groups) {
    for (size_t start = 0; start + 1 < members.size(); start += FH_GEMM_MAX_GROUPS) {
      const size_t count = std::min<size_t>(FH_GEMM_MAX_GROUPS, members.size() - start);
      if (count < 2) break;
      std::vector<Member> part(members.begin() + static_cast<std::ptrdiff_t>(start),
                               members.begin() + static_cast<std::ptrdiff_t>(start + count));
      const size_t first = part.front().pos;
      bool ok = true;
      for (const Member& m : part)
        for (const ir::Value* v : m.node->inputs())
          if (v->producer() != nullptr && pos[v->producer()] >= first) ok = false;
      if (!ok) continue;
      std::vector<ir::Value*> ins{part.front().node->inputs()[0]};
      for (const Member& m : part) ins.push_back(m.node->inputs()[1]);
      for (const Member& m : part)
        for (size_t j = 2; j < m.node->inputs().size(); ++j) ins.push_back(m.node->inputs()[j]);
      std::vector<ir::TensorType> types;
      for (const Member& m : part) types.push_back(m.node->outputs()[0].type());
      Result<ir::Node*> f = g.create_node(std::string(kGemmGroupedOp), ins, types);
      if (!f.is_ok()) return f.status();
      f.value()->set_attr("groups", ir::AttrValue{static_cast<int64_t>(count)});
      f.value()->set_attr("ep_ops", ir::AttrValue{program(part.front().node)});
      f.value()->set_attr("any_order", ir::AttrValue{int64_t{1}});
      // Every operand of the merged node is produced before its first member, so it can stand at that position:
      // a later group reading one of its outputs compares against that position, not against a missing entry.
      pos[f.value()] = first;
      for (size_t i = 0; i < count; ++i) {
        FRAME_RETURN_IF_ERROR(g.replace_all_uses(part[i].node->output(0), f.value()->output(static_cast<int32_t>(i))));
        FRAME_RETURN_IF_ERROR(g.erase_node(part[i].node));
      }
    }
  }
  return Status::ok();
}

Result<ir::Graph> lower_for_hip(const ir::Graph& graph, int32_t opt_level) {
  Result<ir::Graph> work = lower_matmul_grads(graph);
  if (!work.is_ok()) return work.status();
  // Attention runs at every level (like the conv lowering), before the epilogue fusion would claim its matmuls.
  FRAME_RETURN_IF_ERROR(lower_attention(work.value()));
  if (opt_level >= 1) FRAME_RETURN_IF_ERROR(lower_relu_grads(work.value()));
  if (opt_level >= 1) FRAME_RETURN_IF_ERROR(lower_pool_relu_grads(work.value()));
  if (opt_level >= 1) FRAME_RETURN_IF_ERROR(lower_masked_adds(work.value()));
  if (opt_level >= 1) FRAME_RETURN_IF_ERROR(lower_epilogues(work.value()));
  if (opt_level >= 1) FRAME_RETURN_IF_ERROR(lower_gemm_softmax(work.value()));
  if (opt_level >= 1) FRAME_RETURN_IF_ERROR(lower_grouped_gemms(work.value()));
  if (opt_level >= 1) FRAME_RETURN_IF_ERROR(lower_scaled_adds(work.value()));
  FRAME_RETURN_IF_ERROR(lower_stem_pools(work.value()));
  // Channels-last conv lowering runs at every level, so the conv numerics do not depend on the level.
  return lower_convs(work.value());
}

Status hip_run_tapped(hal::Executable& exe, std::span<const Tensor> inputs, std::span<Tensor> outputs, hal::Stream& stream,
                      std::span<const HipStepTap> taps) {
  return static_cast<HipExecutable&>(exe).run_tapped(inputs, outputs, stream, taps);
}

std::string hip_executable_steps(const hal::Executable& exe) { return static_cast<const HipExecutable&>(exe).step_list(); }

Result<std::unique_ptr<hal::Executable>> compile_hip_executable(const ir::Graph& graph, const hal::CompileOptions& options,
                                                                 HipAllocator& allocator, Device device) {
  Result<ir::Graph> lowered = lower_for_hip(graph, options.opt_level);
  if (!lowered.is_ok()) return lowered.status();
  Result<ops::ExecutablePlan> plan = ops::build_executable_plan(lowered.value(), kHipBackendName);
  if (!plan.is_ok()) return plan.status();
  auto exe = std::make_unique<HipExecutable>(std::move(plan.value()), allocator, device, options);
  FRAME_RETURN_IF_ERROR(exe->materialize_constants());
  return std::unique_ptr<hal::Executable>(std::move(exe));
}

}  // namespace frame::backends::hip

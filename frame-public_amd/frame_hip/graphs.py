"""Frame IR builders for the five benchmark configurations, emitted as IR text (the dump_text format).

Graph shapes follow the reference's own factories so that the compiled graphs are the ones Frame builds:
Linear = matmul(x, W) then add(., bias[batch, out]) (reference: src/nn/layers.cpp:238-270); multi-head
attention is unrolled per (batch, head) into slice/transpose/matmul/mul(constant 1/sqrt(dh))/softmax/matmul
and concatenated per batch then across batches (reference: src/nn/layers.cpp:1014-1080). The transformer block
is pre-LN with GELU as BASELINE.json specifies (the reference's own block is post-LN + ReLU,
src/nn/layers.cpp:1099-1172); residual adds are written add(sublayer_out, residual) so the fusion pass chains
them. ResNet-18 uses conv2d with bias for folded batch norm.
"""
from __future__ import annotations

import math

import numpy as np

from . import synth

F32, F16, BF16 = 0, 2, 3
DTYPE_NAME = {F32: "float32", F16: "float16", BF16: "bfloat16"}


def _fmt_double(x: float) -> str:
    s = repr(float(x))
    return s if any(c in s for c in ".eEn") else s + ".0"


def _fmt_attr(v) -> str:
    if isinstance(v, bool):
        return "true" if v else "false"
    if isinstance(v, int):
        return str(v)
    if isinstance(v, float):
        return _fmt_double(v)
    if isinstance(v, str):
        return '"' + v.replace("\\", "\\\\").replace('"', '\\"').replace("\n", "\\n") + '"'
    if isinstance(v, Shape):
        return "shape[" + ",".join(str(d) for d in v.dims) + "]"
    if isinstance(v, DType):
        return f"dtype({DTYPE_NAME[v.code]})"
    if isinstance(v, (list, tuple)):
        if any(isinstance(e, float) for e in v):
            return "[" + ", ".join(_fmt_double(e) for e in v) + "]"
        return "[" + ", ".join(str(int(e)) for e in v) + "]"
    raise TypeError(type(v))


class Shape:
    def __init__(self, dims):
        self.dims = tuple(int(d) for d in dims)


class DType:
    def __init__(self, code):
        self.code = code


class Val:
    def __init__(self, vid, dtype, shape):
        self.id, self.dtype, self.shape = vid, dtype, tuple(shape)


class Graph:
    """Append-only IR text builder; values are numbered in creation order (a topological order)."""

    def __init__(self, device: str = "hip"):
        self.device = device
        self.lines: list[str] = []
        self.outputs: list[Val] = []
        self.next = 0
        self.inputs: list[Val] = []

    def _type(self, dtype, shape):
        return f"{DTYPE_NAME[dtype]}[{','.join(str(d) for d in shape)}]@{self.device}:0"

    def input(self, dtype, shape) -> Val:
        v = Val(self.next, dtype, shape)
        self.next += 1
        self.lines.append(f"%{v.id} = graph_input() : {self._type(dtype, shape)}")
        self.inputs.append(v)
        return v

    def op(self, name, inputs, shape, attrs=None, dtype=None) -> Val:
        dtype = inputs[0].dtype if dtype is None else dtype
        v = Val(self.next, dtype, shape)
        self.next += 1
        text = f"%{v.id} = {name}({', '.join('%' + str(i.id) for i in inputs)})"
        if attrs:
            text += " {" + ", ".join(f"{k}={_fmt_attr(attrs[k])}" for k in sorted(attrs)) + "}"
        self.lines.append(text + " : " + self._type(dtype, shape))
        return v

    def output(self, v: Val) -> None:
        self.outputs.append(v)

    def text(self) -> str:
        return "\n".join(self.lines + [f"graph_output(%{v.id})" for v in self.outputs]) + "\n"

    # ---- op helpers with shape rules -------------------------------------------------------------------------
    def matmul(self, a, b):
        return self.op("matmul", [a, b], (a.shape[0], b.shape[1]))

    def add(self, a, b):
        return self.op("add", [a, b], a.shape)

    def mul(self, a, b):
        return self.op("mul", [a, b], a.shape)

    def relu(self, a):
        return self.op("relu", [a], a.shape)

    def gelu(self, a):
        return self.op("gelu", [a], a.shape)

    def softmax(self, a):
        return self.op("softmax", [a], a.shape)

    def layer_norm(self, x, g, b, eps=1e-5):
        return self.op("layer_norm", [x, g, b], x.shape, {"eps": float(eps)})

    def conv2d(self, x, w, b=None, stride=(1, 1), padding=(0, 0), groups=1):
        n, _, h, wd = x.shape
        cout, _, kh, kw = w.shape
        oh = (h + 2 * padding[0] - kh) // stride[0] + 1
        ow = (wd + 2 * padding[1] - kw) // stride[1] + 1
        ins = [x, w] + ([b] if b is not None else [])
        return self.op("conv2d", ins, (n, cout, oh, ow),
                       {"stride": list(stride), "padding": list(padding), "groups": int(groups)})

    def pool(self, kind, x, kernel, stride, padding):
        n, c, h, w = x.shape
        oh = (h + 2 * padding[0] - kernel[0]) // stride[0] + 1
        ow = (w + 2 * padding[1] - kernel[1]) // stride[1] + 1
        return self.op(kind, [x], (n, c, oh, ow),
                       {"kernel": list(kernel), "stride": list(stride), "padding": list(padding)})

    def reshape(self, x, shape):
        return self.op("reshape", [x], shape, {"target_shape": Shape(shape)})

    def transpose(self, x, perm):
        return self.op("transpose", [x], tuple(x.shape[p] for p in perm), {"perm": list(perm)})

    def slice(self, x, axis, start, stop):
        shape = list(x.shape)
        shape[axis] = stop - start
        return self.op("slice", [x], shape, {"axis": axis, "start": start, "stop": stop})

    def concat(self, xs, axis):
        shape = list(xs[0].shape)
        shape[axis] = sum(x.shape[axis] for x in xs)
        return self.op("concat", xs, shape, {"axis": axis})

    def mse_loss(self, pred, target):
        return self.op("mse_loss", [pred, target], ())

    def sum(self, x, axes, keepdims=False):
        red = set(range(len(x.shape))) if not axes else set(axes)
        shape = tuple((1 if keepdims else None) if i in red else d for i, d in enumerate(x.shape))
        attrs = {"axes": list(axes)}
        if keepdims:
            attrs["keepdims"] = True
        return self.op("sum", [x], tuple(d for d in shape if d is not None), attrs)

    def square(self, a):
        return self.op("square", [a], a.shape)

    def constant_splat(self, dtype, shape, value):
        n = int(np.prod(shape))
        return self.op("constant", [], shape, {"value": [float(value)] * n, "shape": Shape(shape), "dtype": DType(dtype)},
                       dtype=dtype)


# ---- C1: tiny MLP ---------------------------------------------------------------------------------------------

def mlp(batch=64, dtype=F32, device="hip"):
    g = Graph(device)
    x = g.input(dtype, (batch, 784))
    w1 = g.input(dtype, (784, 256))
    b1 = g.input(dtype, (batch, 256))
    w2 = g.input(dtype, (256, 10))
    b2 = g.input(dtype, (batch, 10))
    h = g.relu(g.add(g.matmul(x, w1), b1))
    y = g.softmax(g.add(g.matmul(h, w2), b2))
    g.output(y)
    return g


def mlp_inputs(batch=64, dtype=F32, seed=1):
    return [synth.tensor(seed, (batch, 784), dtype, "normal"),
            synth.tensor(seed + 1, (784, 256), dtype, "normal", math.sqrt(2.0 / 784)),
            synth.tensor(0, (batch, 256), dtype, "zeros"),
            synth.tensor(seed + 2, (256, 10), dtype, "normal", math.sqrt(2.0 / 256)),
            synth.tensor(0, (batch, 10), dtype, "zeros")]


def mlp_train(batch=64, dtype=F32, device="hip", hidden=256, classes=10, features=784):
    """C1's MLP as a training objective: mse_loss(logits, target). Inputs x, w1, b1, w2, b2, target; output the loss.
    The parameters are graph inputs 1..4 (the wrt list of the backward graph)."""
    g = Graph(device)
    x = g.input(dtype, (batch, features))
    w1 = g.input(dtype, (features, hidden))
    b1 = g.input(dtype, (batch, hidden))
    w2 = g.input(dtype, (hidden, classes))
    b2 = g.input(dtype, (batch, classes))
    t = g.input(dtype, (batch, classes))
    h = g.relu(g.add(g.matmul(x, w1), b1))
    g.output(g.mse_loss(g.add(g.matmul(h, w2), b2), t))
    return g


def mlp_train_inputs(batch=64, dtype=F32, seed=11, hidden=256, classes=10, features=784):
    return [synth.tensor(seed, (batch, features), dtype, "normal"),
            synth.tensor(seed + 1, (features, hidden), dtype, "normal", math.sqrt(2.0 / features)),
            synth.tensor(seed + 2, (batch, hidden), dtype, "normal", 0.1),
            synth.tensor(seed + 3, (hidden, classes), dtype, "normal", math.sqrt(2.0 / hidden)),
            synth.tensor(seed + 4, (batch, classes), dtype, "normal", 0.1),
            synth.tensor(seed + 5, (batch, classes), dtype, "normal")]


def cnn_train(batch=8, dtype=F32, device="hip", cin=3, image=32, c1=32, c2=64, classes=10):
    """A small CNN training objective over every gradient-path op: conv+bias, relu, 3x3/s2 max pool, strided conv,
    residual add, square, global avg pool, reshape, matmul, add, mse_loss. Parameters are inputs 1..7."""
    g = Graph(device)
    x = g.input(dtype, (batch, cin, image, image))
    w1 = g.input(dtype, (c1, cin, 3, 3))
    b1 = g.input(dtype, (c1,))
    w2 = g.input(dtype, (c2, c1, 3, 3))
    w3 = g.input(dtype, (c2, c2, 1, 1))
    wf = g.input(dtype, (c2, classes))
    bf = g.input(dtype, (batch, classes))
    scale = g.input(dtype, (batch, c2, image // 4, image // 4))
    t = g.input(dtype, (batch, classes))
    h = g.relu(g.conv2d(x, w1, b1, stride=(1, 1), padding=(1, 1)))
    h = g.pool("max_pool2d", h, (3, 3), (2, 2), (1, 1))
    h = g.relu(g.conv2d(h, w2, None, stride=(2, 2), padding=(1, 1)))
    r = g.conv2d(h, w3, None, stride=(1, 1), padding=(0, 0))
    h = g.relu(g.add(h, g.mul(g.square(r), scale)))
    s = image // 4
    h = g.pool("avg_pool2d", h, (s, s), (s, s), (0, 0))
    h = g.reshape(h, (batch, c2))
    g.output(g.mse_loss(g.add(g.matmul(h, wf), bf), t))
    return g


def cnn_train_inputs(batch=8, dtype=F32, seed=21, cin=3, image=32, c1=32, c2=64, classes=10):
    s = image // 4
    return [synth.tensor(seed, (batch, cin, image, image), dtype, "normal"),
            synth.tensor(seed + 1, (c1, cin, 3, 3), dtype, "normal", math.sqrt(2.0 / (cin * 9))),
            synth.tensor(seed + 2, (c1,), dtype, "normal", 0.1),
            synth.tensor(seed + 3, (c2, c1, 3, 3), dtype, "normal", math.sqrt(2.0 / (c1 * 9))),
            synth.tensor(seed + 4, (c2, c2, 1, 1), dtype, "normal", math.sqrt(1.0 / c2)),
            synth.tensor(seed + 5, (c2, classes), dtype, "normal", math.sqrt(2.0 / c2)),
            synth.tensor(seed + 6, (batch, classes), dtype, "normal", 0.1),
            synth.tensor(seed + 7, (batch, c2, s, s), dtype, "normal", 0.1),
            synth.tensor(seed + 8, (batch, classes), dtype, "normal")]


# ---- C2: GEMM -------------------------------------------------------------------------------------------------

def gemm(n, dtype, device="hip", m=None, k=None):
    m = n if m is None else m
    k = n if k is None else k
    g = Graph(device)
    a = g.input(dtype, (m, k))
    b = g.input(dtype, (k, n))
    g.output(g.matmul(a, b))
    return g


def gemm_inputs(n, dtype, seed=31, m=None, k=None):
    m = n if m is None else m
    k = n if k is None else k
    return [synth.tensor(seed, (m, k), dtype, "uniform"), synth.tensor(seed + 1, (k, n), dtype, "uniform")]


# ---- C3: conv2d + bias + relu ---------------------------------------------------------------------------------

C3 = dict(n=32, cin=64, h=56, w=56, cout=64, k=3)


def conv(dtype, device="hip", n=32, cin=64, h=56, w=56, cout=64, k=3, stride=1, pad=1):
    g = Graph(device)
    x = g.input(dtype, (n, cin, h, w))
    wt = g.input(dtype, (cout, cin, k, k))
    b = g.input(dtype, (cout,))
    g.output(g.relu(g.conv2d(x, wt, b, (stride, stride), (pad, pad))))
    return g


def conv_inputs(dtype, seed=101, n=32, cin=64, h=56, w=56, cout=64, k=3):
    return [synth.tensor(seed, (n, cin, h, w), dtype, "normal"),
            synth.tensor(seed + 1, (cout, cin, k, k), dtype, "normal", math.sqrt(2.0 / (cin * k * k))),
            synth.tensor(seed + 2, (cout,), dtype, "normal", 0.1)]


# ---- C4: ResNet-18 --------------------------------------------------------------------------------------------

def resnet18(batch=64, dtype=BF16, device="hip", image=224, classes=1000, train=False):
    """Returns (graph, parameter specs [(shape, fan_in or None for bias)] in input order after x). With train=True
    the graph takes one more input, the target [batch, classes], and outputs mse_loss(logits, target); the
    parameters are then graph inputs 1..len(specs)."""
    g = Graph(device)
    specs = []
    x = g.input(dtype, (batch, 3, image, image))

    def param(shape, fan_in):
        specs.append((tuple(shape), fan_in))
        return g.input(dtype, shape)

    def conv_bn(v, cout, k, stride, pad):
        w = param((cout, v.shape[1], k, k), v.shape[1] * k * k)
        b = param((cout,), None)
        return g.conv2d(v, w, b, (stride, stride), (pad, pad))

    h = g.relu(conv_bn(x, 64, 7, 2, 3))
    h = g.pool("max_pool2d", h, (3, 3), (2, 2), (1, 1))
    for stage, cout in enumerate((64, 128, 256, 512)):
        for block in range(2):
            stride = 2 if (stage > 0 and block == 0) else 1
            identity = h
            y = g.relu(conv_bn(h, cout, 3, stride, 1))
            y = conv_bn(y, cout, 3, 1, 1)
            if stride != 1 or identity.shape[1] != cout:
                identity = conv_bn(identity, cout, 1, stride, 0)
            h = g.relu(g.add(y, identity))
    hw = h.shape[2]
    h = g.pool("avg_pool2d", h, (hw, hw), (1, 1), (0, 0))
    h = g.reshape(h, (batch, h.shape[1]))
    w = param((h.shape[1], classes), h.shape[1])
    b = param((batch, classes), None)
    logits = g.add(g.matmul(h, w), b)
    if train:
        g.output(g.mse_loss(logits, g.input(dtype, (batch, classes))))
    else:
        g.output(logits)
    return g, specs


def resnet18_inputs(specs, batch=64, dtype=BF16, image=224, seed=401):
    arrays = [synth.tensor(seed, (batch, 3, image, image), dtype, "normal")]
    for i, (shape, fan_in) in enumerate(specs):
        if fan_in is None:
            arrays.append(synth.tensor(seed + 1 + i, shape, dtype, "normal", 0.01))
        else:
            arrays.append(synth.tensor(seed + 1 + i, shape, dtype, "normal", math.sqrt(2.0 / fan_in)))
    return arrays


# ---- C5: transformer encoder block (pre-LN, GELU) ---------------------------------------------------------------

def transformer_block(batch=8, seq=512, d_model=1024, heads=16, ffn=4096, dtype=BF16, device="hip", act="gelu",
                      train=False):
    """C5's pre-LN block. act selects the FFN activation ("relu" gives a block the reference can also build);
    train=True adds a target input [rows, d_model] after the parameters and outputs mse_loss(y, target)."""
    g = Graph(device)
    rows = batch * seq
    dh = d_model // heads
    x = g.input(dtype, (rows, d_model))
    names = ["ln1_g", "ln1_b", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "ln2_g", "ln2_b", "w1", "b1", "w2", "b2"]
    shapes = [(d_model,), (d_model,), (d_model, d_model), (rows, d_model), (d_model, d_model), (rows, d_model),
              (d_model, d_model), (rows, d_model), (d_model, d_model), (rows, d_model), (d_model,), (d_model,),
              (d_model, ffn), (rows, ffn), (ffn, d_model), (rows, d_model)]
    p = {n: g.input(dtype, s) for n, s in zip(names, shapes)}
    h1 = g.layer_norm(x, p["ln1_g"], p["ln1_b"])
    q = g.add(g.matmul(h1, p["wq"]), p["bq"])
    k = g.add(g.matmul(h1, p["wk"]), p["bk"])
    v = g.add(g.matmul(h1, p["wv"]), p["bv"])
    # One [seq, seq] splat of 1/sqrt(dh) shared by every head: the reference's factory emits one identical
    # constant per (batch, head) and common_subexpression_elimination merges them into exactly this node.
    scale = g.constant_splat(dtype, (seq, seq), 1.0 / math.sqrt(dh))
    per_batch = []
    for b in range(batch):
        qr, kr, vr = (g.slice(t, 0, b * seq, (b + 1) * seq) for t in (q, k, v))
        heads_out = []
        for hd in range(heads):
            qh, kh, vh = (g.slice(t, 1, hd * dh, (hd + 1) * dh) for t in (qr, kr, vr))
            s = g.matmul(qh, g.transpose(kh, (1, 0)))
            s = g.mul(s, scale)
            heads_out.append(g.matmul(g.softmax(s), vh))
        per_batch.append(g.concat(heads_out, 1))
    attn = g.concat(per_batch, 0)
    o = g.add(g.matmul(attn, p["wo"]), p["bo"])
    h = g.add(o, x)
    h2 = g.layer_norm(h, p["ln2_g"], p["ln2_b"])
    pre = g.add(g.matmul(h2, p["w1"]), p["b1"])
    f = g.gelu(pre) if act == "gelu" else g.relu(pre)
    y = g.add(g.add(g.matmul(f, p["w2"]), p["b2"]), h)
    if train:
        g.output(g.mse_loss(y, g.input(dtype, (rows, d_model))))
    else:
        g.output(y)
    return g, shapes


def transformer_inputs(shapes, rows=4096, d_model=1024, dtype=BF16, seed=501):
    arrays = [synth.tensor(seed, (rows, d_model), dtype, "normal")]
    for i, s in enumerate(shapes):
        if len(s) == 1:  # layer-norm gamma = 1 + noise, beta = noise
            base = synth.tensor(seed + 1 + i, s, F32, "normal", 0.02)
            v = base + (1.0 if i in (0, 10) else 0.0)
            arrays.append(synth.to_storage(v.astype(np.float32), dtype))
        elif s[0] == rows:  # full-shape biases are zero (the reference's Linear bias is [batch, out])
            arrays.append(synth.tensor(0, s, dtype, "zeros"))
        else:
            arrays.append(synth.tensor(seed + 1 + i, s, dtype, "normal", 0.02))
    return arrays

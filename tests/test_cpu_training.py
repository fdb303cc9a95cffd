"""Training path, host side (no GPU): the training-graph construction and the oracle's gradient kernels.

* build_backward_graph / build_sgd_update_graph on IR text: identical text to the reference's own autograd
  (oracle/_ref, the reference compiled from its sources), before and after the standard pipeline, and the same
  error codes for the reference's rejection cases (src/compiler/autograd.cpp:118-300).
* The oracle's restatement of every gradient-only op (oracle/cpu_kernels.cpp, training section): bit-identical to
  the reference build on seeded inputs, per op and through whole training graphs.
* Independent pins from the mathematics (no reference code involved): each gradient op is the adjoint of its
  forward linear map, <f(x), y> = <x, f^T(y)>, checked in float64 on the oracle's float32 outputs; the max-pool
  gradient against a numpy scatter with numpy's own argmax; mse_loss and its gradient against their closed forms;
  the backward of the MLP against central finite differences of the loss.
"""
import re

import numpy as np
import pytest

import oracle_lib as orc
from frame_hip import graphs, host, synth

F32, F16, BF16 = 0, 2, 3
needs_ref = pytest.mark.skipif(not orc.ref_available(), reason="reference build (oracle/_ref) not present")


@pytest.fixture(autouse=True)
def _cpu_backend():
    orc.load_cpu_backend()  # the oracle's `cpu` backend: the pipeline's backend_lowering pass needs it registered


def cpu_graph(name, in_shapes, out_shape, attrs=None, dtype=F32):
    g = graphs.Graph("cpu")
    vals = [g.input(dtype, s) for s in in_shapes]
    g.output(g.op(name, vals, out_shape, attrs))
    return g.text()


def run(text, ins):
    return orc.run_graph_cpu(text, ins)


def run_ref(text, ins, outs):
    return orc.ref_run_graph(text, ins, outs)


def bits(a):
    return np.ascontiguousarray(a).reshape(-1).view(np.uint8)


# ---- graph construction -------------------------------------------------------------------------------------

GRAPHS = [("mlp", graphs.mlp_train, dict(batch=4), [1, 2, 3, 4]),
          ("cnn", graphs.cnn_train, dict(batch=2, image=16), [1, 2, 3, 4, 5, 6]),
          ("cnn-partial", graphs.cnn_train, dict(batch=2, image=16), [6, 0, 2])]


@needs_ref
@pytest.mark.parametrize("dtype", [F32, BF16, F16])
@pytest.mark.parametrize("name,mk,kw,wrt", GRAPHS)
def test_backward_graph_text_matches_reference(name, mk, kw, wrt, dtype):
    fwd = mk(dtype=dtype, device="cpu", **kw).text()
    mine = host.backward(fwd, 0, wrt)
    assert mine == orc.ref_backward(fwd, 0, wrt)
    # and after the nine-pass pipeline (fusion, CSE, dead nodes, memory plan)
    assert host.transform(mine) == orc.ref_transform(mine)


@needs_ref
def test_sgd_graph_text_matches_reference():
    fwd = graphs.cnn_train(dtype=BF16, device="cpu", batch=2, image=16).text()
    for lr in (0.1, 1e-3):
        assert host.sgd_update(fwd, [1, 2, 3], lr) == orc.ref_sgd_update(fwd, [1, 2, 3], lr)


def test_unreached_wrt_input_gets_zero_gradient():
    fwd = graphs.mlp_train(batch=2, features=3, hidden=4, classes=2, device="cpu").text()
    text = host.backward(fwd, 0, [5])  # the target: reached (mse_loss is differentiable in it)
    assert "mse_loss_grad_internal" in text
    g = graphs.Graph("cpu")
    x = g.input(F32, (2, 3))
    g.input(F32, (3, 3))  # unused input
    g.output(g.mse_loss(x, x))
    text = host.backward(g.text(), 0, [1])
    assert "value=[0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0]" in text


@needs_ref
@pytest.mark.parametrize("case", ["nonscalar", "loss_range", "wrt_range", "wrt_dup", "no_gradient"])
def test_backward_errors_match_reference(case):
    g = graphs.Graph("cpu")
    x = g.input(F32, (4, 8))
    w = g.input(F32, (8, 3))
    y = g.matmul(x, w)
    if case == "no_gradient":  # fused_elementwise_internal has no GradientFn in either build
        g.output(g.sum(g.op("fused_elementwise_internal", [y], y.shape, {"ops": "relu", "arities": [1]}), []))
    elif case == "nonscalar":
        g.output(y)
    else:
        g.output(g.sum(y, []))
    loss, wrt = {"loss_range": (1, [1]), "wrt_range": (0, [2]), "wrt_dup": (0, [1, 1])}.get(case, (0, [1]))
    with pytest.raises(host.FrameError) as mine:
        host.backward(g.text(), loss, wrt)
    with pytest.raises(RuntimeError) as ref:
        orc.ref_backward(g.text(), loss, wrt)
    import re
    ref_code = int(re.search(r"reference call failed \((\d+)\)", str(ref.value)).group(1))
    assert mine.value.code == ref_code  # frame::ErrorCode ordinals on both sides
    assert ref_code == (host.CODES["unimplemented"] if case == "no_gradient" else host.CODES["invalid_argument"])


# ---- oracle vs the reference build -----------------------------------------------------------------------------

@needs_ref
@pytest.mark.parametrize("dtype", [F32, BF16, F16])
@pytest.mark.parametrize("name,mk,kw,wrt", GRAPHS[:2])
def test_oracle_training_graph_bit_identical_to_reference(name, mk, kw, wrt, dtype):
    fwd = mk(dtype=dtype, device="cpu", **kw).text()
    text = host.backward(fwd, 0, wrt)
    ins = (graphs.mlp_train_inputs if name == "mlp" else graphs.cnn_train_inputs)(dtype=dtype, **kw)
    mine = run(text, ins)
    ref = run_ref(text, ins, [(o.shape, o.dtype) for o in mine])
    for i, (a, b) in enumerate(zip(mine, ref)):
        assert np.array_equal(bits(a), bits(b)), f"output {i}"


OP_CASES = [
    ("relu_grad_internal", [(5, 33), (5, 33)], (5, 33), None),
    ("matmul_grad_lhs_internal", [(7, 5), (9, 5)], (7, 9), None),
    ("matmul_grad_rhs_internal", [(7, 9), (7, 5)], (9, 5), None),
    ("conv2d_grad_input_internal", [(2, 6, 4, 5), (6, 4, 3, 3)], (2, 4, 8, 9),
     {"input_shape": graphs.Shape((2, 4, 8, 9)), "stride": [2, 2], "padding": [1, 1], "groups": 1}),
    ("conv2d_grad_filter_internal", [(2, 4, 8, 9), (2, 6, 4, 5)], (6, 4, 3, 3),
     {"filter_shape": graphs.Shape((6, 4, 3, 3)), "stride": [2, 2], "padding": [1, 1], "groups": 1}),
    ("conv2d_grad_input_internal", [(2, 6, 8, 8), (6, 2, 3, 3)], (2, 4, 8, 8),
     {"input_shape": graphs.Shape((2, 4, 8, 8)), "stride": [1, 1], "padding": [1, 1], "groups": 2}),
    ("max_pool2d_grad_internal", [(2, 3, 5, 5), (2, 3, 9, 9)], (2, 3, 9, 9),
     {"input_shape": graphs.Shape((2, 3, 9, 9)), "kernel": [3, 3], "stride": [2, 2], "padding": [1, 1]}),
    ("avg_pool2d_grad_internal", [(2, 3, 5, 5)], (2, 3, 9, 9),
     {"input_shape": graphs.Shape((2, 3, 9, 9)), "kernel": [3, 3], "stride": [2, 2], "padding": [1, 1]}),
    ("sum", [(3, 4, 5, 6)], (4,), {"axes": [0, 2, 3]}),
    ("sum", [(3, 4, 5)], (1, 4, 1), {"axes": [0, 2], "keepdims": True}),
    ("sum", [(300, 7)], (), {"axes": []}),
    ("sum_grad_internal", [(4,)], (3, 4, 5, 6), {"axes": [0, 2, 3], "input_shape": graphs.Shape((3, 4, 5, 6))}),
    ("mse_loss", [(33, 7), (33, 7)], (), None),
    ("mse_loss_grad_internal", [(33, 7), (33, 7), ()], (33, 7), None),
]


@needs_ref
@pytest.mark.parametrize("dtype", [F32, BF16, F16])
@pytest.mark.parametrize("case", OP_CASES, ids=lambda c: c[0] + str(c[2]))
def test_oracle_op_bit_identical_to_reference(case, dtype):
    name, ins_s, out_s, attrs = case
    text = cpu_graph(name, ins_s, out_s, attrs, dtype)
    ins = [synth.tensor(90 + i, s, dtype).reshape(s) for i, s in enumerate(ins_s)]
    if name.startswith("max_pool"):
        ins[1].reshape(-1)[::5] = ins[1].reshape(-1)[2]  # ties
    (mine,) = run(text, ins)
    (ref,) = run_ref(text, ins, [(mine.shape, mine.dtype)])
    assert np.array_equal(bits(mine), bits(ref))


# ---- pins from the mathematics ---------------------------------------------------------------------------------

def f64(a):
    return np.asarray(a, dtype=np.float64)


def conv_ref64(x, w, s, p):
    """float64 direct convolution (groups 1), written from the definition."""
    n, cin, h, wd = x.shape
    cout, _, kh, kw = w.shape
    oh, ow = (h + 2 * p - kh) // s + 1, (wd + 2 * p - kw) // s + 1
    xp = np.zeros((n, cin, h + 2 * p, wd + 2 * p))
    xp[:, :, p:p + h, p:p + wd] = x
    y = np.zeros((n, cout, oh, ow))
    for a in range(kh):
        for b in range(kw):
            patch = xp[:, :, a:a + s * oh:s, b:b + s * ow:s]  # [n, cin, oh, ow]
            y += np.einsum("nchw,oc->nohw", patch, w[:, :, a, b])
    return y


@pytest.mark.parametrize("s,p,k", [(1, 1, 3), (2, 1, 3), (2, 0, 1), (2, 3, 7)])
def test_conv_grads_are_adjoints(s, p, k):
    rng = np.random.default_rng(5)
    n, cin, h, w, cout = 2, 3, 11, 10, 4
    x = rng.standard_normal((n, cin, h, w)).astype(np.float32)
    wt = rng.standard_normal((cout, cin, k, k)).astype(np.float32)
    y = conv_ref64(f64(x), f64(wt), s, p)
    dy = rng.standard_normal(y.shape).astype(np.float32)
    common = {"stride": [s, s], "padding": [p, p], "groups": 1}
    (gx,) = run(cpu_graph("conv2d_grad_input_internal", [dy.shape, wt.shape], x.shape,
                          dict(common, input_shape=graphs.Shape(x.shape))), [dy, wt])
    (gw,) = run(cpu_graph("conv2d_grad_filter_internal", [x.shape, dy.shape], wt.shape,
                          dict(common, filter_shape=graphs.Shape(wt.shape))), [x, dy])
    lhs = np.sum(y * f64(dy))
    np.testing.assert_allclose(np.sum(f64(x) * f64(gx)), lhs, rtol=1e-5)
    np.testing.assert_allclose(np.sum(f64(wt) * f64(gw)), lhs, rtol=1e-5)


def test_avg_pool_grad_is_adjoint_and_max_pool_grad_scatters_to_argmax():
    rng = np.random.default_rng(6)
    xs, k, s, p = (2, 3, 9, 8), 3, 2, 1
    x = rng.standard_normal(xs).astype(np.float32)
    oh, ow = (9 + 2 * p - k) // s + 1, (8 + 2 * p - k) // s + 1
    dy = rng.standard_normal((2, 3, oh, ow)).astype(np.float32)
    attrs = {"kernel": [k, k], "stride": [s, s], "padding": [p, p], "input_shape": graphs.Shape(xs)}
    (ga,) = run(cpu_graph("avg_pool2d_grad_internal", [dy.shape], xs, attrs), [dy])
    xp = np.zeros((2, 3, 9 + 2 * p, 8 + 2 * p))
    xp[:, :, p:p + 9, p:p + 8] = x
    avg = np.zeros(dy.shape)
    for a in range(k):
        for b in range(k):
            avg += xp[:, :, a:a + s * oh:s, b:b + s * ow:s]
    avg /= k * k
    np.testing.assert_allclose(np.sum(f64(x) * f64(ga)), np.sum(avg * f64(dy)), rtol=1e-5)
    (gm,) = run(cpu_graph("max_pool2d_grad_internal", [dy.shape, xs], xs, attrs), [dy, x])
    want = np.zeros(xs)
    for nn in range(2):
        for c in range(3):
            for i in range(oh):
                for j in range(ow):
                    h0, w0 = i * s - p, j * s - p
                    hs, ws = max(h0, 0), max(w0, 0)
                    win = x[nn, c, hs:h0 + k, ws:w0 + k]
                    r, q = np.unravel_index(np.argmax(win), win.shape)  # first maximum in row-major order
                    want[nn, c, hs + r, ws + q] += dy[nn, c, i, j]
    np.testing.assert_allclose(f64(gm), want, rtol=1e-6, atol=1e-6)


def test_matmul_sum_and_mse_closed_forms():
    rng = np.random.default_rng(7)
    m, n, k = 9, 5, 7
    gy = rng.standard_normal((m, n)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    a = rng.standard_normal((m, k)).astype(np.float32)
    (ga,) = run(cpu_graph("matmul_grad_lhs_internal", [(m, n), (k, n)], (m, k)), [gy, b])
    (gb,) = run(cpu_graph("matmul_grad_rhs_internal", [(m, k), (m, n)], (k, n)), [a, gy])
    np.testing.assert_allclose(ga, f64(gy) @ f64(b).T, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(gb, f64(a).T @ f64(gy), rtol=1e-5, atol=1e-5)
    x = rng.standard_normal((3, 4, 5, 6)).astype(np.float32)
    (sx,) = run(cpu_graph("sum", [x.shape], (4,), {"axes": [0, 2, 3]}), [x])
    np.testing.assert_allclose(sx, f64(x).sum(axis=(0, 2, 3)), rtol=1e-5, atol=1e-5)
    g = rng.standard_normal((4,)).astype(np.float32)
    (gx,) = run(cpu_graph("sum_grad_internal", [(4,)], x.shape, {"axes": [0, 2, 3], "input_shape": graphs.Shape(x.shape)}), [g])
    assert np.array_equal(gx, np.broadcast_to(g.reshape(1, 4, 1, 1), x.shape))
    pr, t = rng.standard_normal((33, 7)).astype(np.float32), rng.standard_normal((33, 7)).astype(np.float32)
    (loss,) = run(cpu_graph("mse_loss", [pr.shape, t.shape], ()), [pr, t])
    np.testing.assert_allclose(float(loss), np.mean((f64(pr) - f64(t)) ** 2), rtol=1e-5)
    gyl = np.array(0.75, dtype=np.float32)
    (gp,) = run(cpu_graph("mse_loss_grad_internal", [pr.shape, t.shape, ()], pr.shape), [pr, t, gyl])
    np.testing.assert_allclose(gp, 2 * 0.75 / pr.size * (f64(pr) - f64(t)), rtol=1e-5, atol=1e-7)


def test_mlp_backward_matches_finite_differences():
    kw = dict(batch=3, features=5, hidden=6, classes=4)
    fwd = graphs.mlp_train(device="cpu", **kw).text()
    ins = graphs.mlp_train_inputs(**kw)
    ins = [i.astype(np.float32) for i in ins]
    grads = run(host.backward(fwd, 0, [1, 2, 3, 4]), ins)[1:]
    rng = np.random.default_rng(8)
    eps = 1e-2
    for pi, g in zip([1, 2, 3, 4], grads):
        for _ in range(3):
            idx = tuple(rng.integers(0, d) for d in ins[pi].shape)
            plus = [i.copy() for i in ins]
            minus = [i.copy() for i in ins]
            plus[pi][idx] += eps
            minus[pi][idx] -= eps
            fd = (float(run(fwd, plus)[0]) - float(run(fwd, minus)[0])) / (2 * eps)
            assert abs(fd - float(g[idx])) <= 2e-3 * max(1.0, abs(fd)), (pi, idx, fd, float(g[idx]))


@pytest.mark.parametrize("dtype", [F32, BF16])
def test_grad_input_lowering(dtype):
    """conv2d_grad_input_internal becomes flip(w) + channels-last dy (dilated by the stride) + a stride-1 NHWC conv
    with padding K-1-pad where the implicit-GEMM kernel takes the geometry; groups > 1 keeps the direct kernel."""
    def lowered(xs, ws, s, p, groups=1):
        oh, ow = (xs[2] + 2 * p - ws[2]) // s + 1, (xs[3] + 2 * p - ws[3]) // s + 1
        g = graphs.Graph("hip")
        a, b = g.input(dtype, (xs[0], ws[0], oh, ow)), g.input(dtype, ws)
        g.output(g.op("conv2d_grad_input_internal", [a, b], xs,
                      {"input_shape": graphs.Shape(xs), "stride": [s, s], "padding": [p, p], "groups": groups}))
        return host.hip_lowered(g.text())
    t = lowered((8, 64, 56, 56), (128, 64, 3, 3), 2, 1)
    assert "hip_dilate_nhwc_internal(%0) {stride=[2, 2]}" in t and "bfloat16[8,56,56,128]" in t.replace("float32", "bfloat16")
    assert "padding=[1, 1], stride=[1, 1]" in t and "hip_conv_filter_flip_internal" in t
    t = lowered((8, 64, 56, 56), (64, 64, 3, 3), 1, 1)
    assert "hip_channels_last_internal(%0)" in t and "hip_dilate_nhwc_internal" not in t
    t = lowered((8, 64, 57, 57), (128, 64, 1, 1), 2, 0)  # odd size: one trailing zero row/column in the dilation
    assert "[8,57,57,128]" in t
    assert "conv2d_grad_input_internal" in lowered((8, 64, 56, 56), (64, 32, 3, 3), 1, 1, groups=2)


def test_relu_grad_reads_the_relu_output():
    """relu_grad_internal(x, gy) keeps gy where x > 0, and relu(x) > 0 exactly where x > 0, so the lowering gives
    relu_grad the relu's output: the residual block's conv -> add -> relu then becomes one add;relu conv epilogue,
    and both gradients read it. The oracle check: on every bf16 bit pattern, relu_grad over relu(x) equals
    relu_grad over x (NaN, -0, infinities and denormals included)."""
    g = graphs.Graph("hip")
    x, w, b = g.input(BF16, (2, 64, 8, 8)), g.input(BF16, (64, 64, 3, 3)), g.input(BF16, (64,))
    skip, gy, w2 = g.input(BF16, (2, 64, 8, 8)), g.input(BF16, (2, 64, 8, 8)), g.input(BF16, (64, 64, 3, 3))
    c = g.op("conv2d", [x, w, b], (2, 64, 8, 8), {"stride": [1, 1], "padding": [1, 1], "groups": 1})
    a = g.add(c, skip)
    r = g.relu(a)
    g.output(g.op("conv2d", [r, w2], (2, 64, 8, 8), {"stride": [1, 1], "padding": [1, 1], "groups": 1}))
    g.output(g.op("relu_grad_internal", [a, gy], (2, 64, 8, 8), {}))
    g.output(g.op("relu_grad_internal", [r, gy], (2, 64, 8, 8), {}))
    low = host.hip_lowered(g.text(), 1)
    fused = re.search(r"(%\d+) = hip_conv2d_nhwc_internal\([^)]*\) \{ep_ops=\[1, 3\]", low)
    assert fused is not None, low
    grads = re.findall(r"= relu_grad_internal\((%\d+), ", low)
    assert grads == [fused.group(1)] * 2, low
    # at opt level 0 the graph keeps the reference's nodes
    assert "= relu(" in host.hip_lowered(g.text(), 0)
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    gy = np.random.default_rng(3).permutation(bits)
    relu = orc.ew_program(BF16, [3], [1], [bits])
    assert np.array_equal(orc.ew_program(BF16, [6], [2], [bits, gy]), orc.ew_program(BF16, [6], [2], [relu, gy]))
    assert np.count_nonzero(orc.ew_program(BF16, [6], [2], [bits, gy]) != 0) > 30000  # gy passed where x > 0


def test_resnet_training_graph_stays_channels_last():
    """The backward of ResNet-18 reads and writes channels-last activations: conv gradients take NHWC x / dy, the
    transposed convolutions write NHWC, relu_grad / add / bias sums run on NHWC, the global average-pool gradient
    has an NHWC kernel. What is left NCHW is the stem (its max-pool gradient kernel is NCHW) and graph inputs."""
    g, specs = graphs.resnet18(batch=8, dtype=BF16, image=64, train=True)
    low = host.hip_lowered(host.backward(g.text(), 0, list(range(1, len(specs) + 1))), 1)
    assert low.count("hip_channels_last_internal(") <= 13, low.count("hip_channels_last_internal(")
    assert "hip_avg_pool2d_grad_nhwc_internal" in low
    # the 19 input gradients' filters (every conv but the stem) are flipped in one batched step
    assert low.count("hip_conv_filter_flip_multi_internal(") == 1 and "hip_conv_filter_flip_internal(" not in low
    # relu_grad reads the relus' outputs, so every forward relu fuses into its conv as in the inference graph (the
    # eight residual blocks as add;relu) and the stem's input is packed once for the conv and its filter gradient
    ops = re.findall(r"= (\w+)\(", low)
    assert "relu" not in ops
    # seven residual outputs' gradients (the sum of their two consumers' gradients, then the relu mask) are one
    # add-then-mask program each; the eighth block output's sum feeds the stem's pool gradient
    assert ops.count("hip_ew_program_internal") == 7 and low.count("ew_ops=[1, 11]") == 7
    assert ops.count("relu_grad_internal") == 9 and ops.count("add") == 1
    # the stem's relu gradient is the max-pool gradient's mask (one launch; the pool input is the relu's output)
    assert ops.count("hip_max_pool2d_relu_grad_internal") == 1 and "max_pool2d_grad_internal" not in ops
    assert low.count("ep_ops=[1, 3]") == 8 and low.count("ep_ops=[3]") == 9
    assert ops.count("hip_pack_input_c8_internal") == 1
    flips = re.search(r"= hip_conv_filter_flip_multi_internal\(([^)]*)\)", low)
    assert flips is not None and len(flips.group(1).split(",")) == 19, low
    assert low.count("hip_conv2d_wgrad_nhwc_internal") == 20
    assert 'in_nhwc=1' in low  # strided grad_input dilates a channels-last dy
    sums = [l for l in low.splitlines() if " = sum(" in l]
    # bias gradients over N, H, W of NHWC data; the stem region (NCHW, next to the max-pool gradient) keeps [0, 2, 3]
    assert len(sums) + low.count("hip_sum_rows_internal") == 17  # 17 biased convs
    assert sum("axes=[0, 1, 2]" in l for l in sums) + low.count("hip_sum_rows_internal") >= 14  # stem region NCHW


TINY_BLOCK = dict(batch=2, seq=8, d_model=16, heads=2, ffn=32)


@needs_ref
@pytest.mark.parametrize("dtype", [F32, BF16])
def test_transformer_training_graph_matches_reference(dtype):
    """softmax, layer_norm, transpose, slice, concat gradients (and rsqrt, matmul broadcasts, sums in their
    micrographs): the training graph of C5's block (relu FFN: the reference has no gelu) has the reference's IR text,
    and the oracle runs it bit-identically to the reference build."""
    g, shapes = graphs.transformer_block(dtype=dtype, device="cpu", act="relu", train=True, **TINY_BLOCK)
    wrt = list(range(1, len(shapes) + 1))
    text = host.backward(g.text(), 0, wrt)
    assert text == orc.ref_backward(g.text(), 0, wrt)
    assert host.transform(text) == orc.ref_transform(text)
    rows = TINY_BLOCK["batch"] * TINY_BLOCK["seq"]
    ins = graphs.transformer_inputs(shapes, rows=rows, d_model=16, dtype=dtype) + [synth.tensor(77, (rows, 16), dtype)]
    mine = run(text, ins)
    ref = run_ref(text, ins, [(o.shape, o.dtype) for o in mine])
    for i, (a, b) in enumerate(zip(mine, ref)):
        assert np.array_equal(bits(a), bits(b)), f"output {i}"


@needs_ref
@pytest.mark.parametrize("op", ["sigmoid", "tanh", "rsqrt"])
def test_unary_ops_and_gradients_match_reference(op):
    g = graphs.Graph("cpu")
    x = g.input(F32, (6, 50))
    y = g.op(op, [x], (6, 50))
    g.output(g.sum(g.mul(y, y), []))
    text = host.backward(g.text(), 0, [0])
    assert text == orc.ref_backward(g.text(), 0, [0])
    xs = np.abs(synth.tensor(5, (6, 50), F32)).astype(np.float32) + (0.1 if op == "rsqrt" else 0.0)
    if op != "rsqrt":
        xs = synth.tensor(5, (6, 50), F32) * 4
    mine = run(text, [xs])
    ref = run_ref(text, [xs], [(o.shape, o.dtype) for o in mine])
    for a, b in zip(mine, ref):
        assert np.array_equal(bits(a), bits(b))


def test_gelu_gradient_matches_the_derivative():
    # gelu has no reference counterpart: its gradient op is pinned by central differences of the exact function
    import math
    xs = np.linspace(-6, 6, 241).astype(np.float32)
    gy = np.ones_like(xs)
    (gx,) = run(cpu_graph("gelu_grad_internal", [xs.shape, xs.shape], xs.shape), [xs, gy])
    def gelu(v):
        return 0.5 * v * (1 + math.erf(v / math.sqrt(2)))
    h = 1e-4
    for v, got in zip(xs.astype(np.float64), gx):
        want = (gelu(v + h) - gelu(v - h)) / (2 * h)
        assert abs(float(got) - want) <= 1e-5 * max(1.0, abs(want)), (v, got, want)
    g = graphs.Graph("cpu")
    x = g.input(F32, (4, 5))
    g.output(g.sum(g.gelu(x), []))
    assert "gelu_grad_internal(%0, " in host.backward(g.text(), 0, [0])


def test_sgd_update_lowers_to_multi_tensor_launches():
    """The SGD update graph's add(param, mul(constant(-lr), grad)) pairs become hip_axpy_multi_internal nodes of
    at most 32 pairs each (42 ResNet-18 parameters: 32 + 10); no mul, add or constant is left. At opt level 0 the
    graph keeps its nodes."""
    g, specs = graphs.resnet18(batch=8, dtype=BF16, image=64, train=True)
    sgd = host.sgd_update(g.text(), list(range(1, len(specs) + 1)), 0.01)
    low = host.hip_lowered(sgd, 1)
    assert low.count("hip_axpy_multi_internal(") == 2, low
    assert " mul(" not in low and " add(" not in low and "constant(" not in low
    assert "scales=[" in low
    assert host.hip_lowered(sgd, 0).count(" mul(") == len(specs)

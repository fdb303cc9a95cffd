"""Training path on the MI355X: the gradient-only ops of compiler::build_backward_graph, each compiled for `hip`
(runtime::compile -> HipBackend::compile -> HipExecutable::run) and compared with the same graph on the oracle's
`cpu` backend, then whole training graphs (backward of an MLP and of a small CNN, and the SGD update graph).

Bit-exact where the hip kernel keeps the reference's per-element summation order (relu_grad, pool gradients, conv
gradients, matmul gradients below the tiled-GEMM threshold, sum_grad, mse_loss_grad); rtol 1e-5 (float32) /
1e-2 (16-bit) with atol = rtol * rms(expected) where the kernel reduces in another order (sum, mse_loss, matmul
gradients on the tiled GEMM) or the graph contains such ops (tests/tolerance.py).
"""
import numpy as np
import pytest

import oracle_lib as orc
from frame_hip import graphs, host, synth
from tolerance import assert_bitwise, assert_close

pytestmark = pytest.mark.gpu
F32, F16, BF16 = 0, 2, 3
DTYPES = [F32, BF16, F16]


def say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def dev():
    assert host.device_count("hip") >= 1, "no hip device"
    orc.load_cpu_backend()


def both(g, ins):
    """(hip outputs, oracle cpu outputs) of graph g (built for device 'hip')."""
    got = host.compile(g.text(), "hip", 1).run(ins)
    want = orc.run_graph_cpu(g.text().replace("@hip:0", "@cpu:0"), ins)
    return got, want


def one_op(name, ins_specs, out_shape, attrs=None, dtype=F32):
    g = graphs.Graph("hip")
    vals = [g.input(dtype, s) for s in ins_specs]
    g.output(g.op(name, vals, out_shape, attrs))
    return g


def tensors(seed, shapes, dtype, kind="normal"):
    return [synth.tensor(seed + i, s, dtype, kind).reshape(s) for i, s in enumerate(shapes)]


def conv_out(h, k, s, p):
    return (h + 2 * p - k) // s + 1


# ---- elementwise ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES)
def test_relu_grad(dev, dtype):
    say(f"relu_grad dtype={dtype}")
    shape = (3, 1000, 17)
    x, gy = tensors(1, [shape, shape], dtype)
    x.reshape(-1)[:40] = 0  # x == 0 takes the zero branch
    got, want = both(one_op("relu_grad_internal", [shape, shape], shape, dtype=dtype), [x, gy])
    assert_bitwise(got[0], want[0], "relu_grad")


# ---- matmul gradients ----------------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,n,k", [(64, 10, 256), (64, 256, 784), (3, 5, 7), (130, 33, 70)])
def test_matmul_grads_small(dev, dtype, m, n, k):
    # below the tiled threshold fh_matmul_grad's sequential kernel reads the transposed operand in place ->
    # bit-exact; above it (16-bit [784,256] here) the backend lowers to transpose + MFMA GEMM -> tolerance
    say(f"matmul_grad small m={m} n={n} k={k} dtype={dtype}")
    gy, b, a = tensors(10, [(m, n), (k, n), (m, k)], dtype)
    for g, ins, what in [(one_op("matmul_grad_lhs_internal", [(m, n), (k, n)], (m, k), dtype=dtype), [gy, b], "lhs"),
                         (one_op("matmul_grad_rhs_internal", [(m, k), (m, n)], (k, n), dtype=dtype), [a, gy], "rhs")]:
        got, want = both(g, ins)
        if "transpose" in host.hip_lowered(g.text()):
            assert_close(got[0], want[0], dtype, what=f"matmul_grad_{what} (tiled)")
        else:
            assert_bitwise(got[0], want[0], f"matmul_grad_{what}")


@pytest.mark.parametrize("dtype", [F32, BF16])
def test_matmul_grads_tiled(dev, dtype):
    # large: lowered to transpose + matmul on the tiled / MFMA GEMM kernels -> tolerance
    m, n, k = 1024, 512, 768
    say(f"matmul_grad tiled dtype={dtype}")
    assert "transpose" in host.hip_lowered(one_op("matmul_grad_lhs_internal", [(m, n), (k, n)], (m, k), dtype=dtype).text())
    gy, b, a = tensors(20, [(m, n), (k, n), (m, k)], dtype)
    got, want = both(one_op("matmul_grad_lhs_internal", [(m, n), (k, n)], (m, k), dtype=dtype), [gy, b])
    assert_close(got[0], want[0], dtype, what="matmul_grad_lhs tiled")
    got, want = both(one_op("matmul_grad_rhs_internal", [(m, k), (m, n)], (k, n), dtype=dtype), [a, gy])
    assert_close(got[0], want[0], dtype, what="matmul_grad_rhs tiled")


def test_matmul_grad_eager_launch(dev):
    say("matmul_grad eager launch")
    m, n, k = 40, 24, 56
    g = one_op("matmul_grad_rhs_internal", [(m, k), (m, n)], (k, n))
    a, gy = tensors(30, [(m, k), (m, n)], F32)
    ta, tg = host.Tensor.from_numpy("hip", F32, a), host.Tensor.from_numpy("hip", F32, gy)
    out = host.Tensor("hip", F32, (k, n))
    s = host.Stream("hip")
    host.launch(g.text(), "hip", [ta, tg], [out], s)
    s.synchronize()
    (want,) = orc.run_graph_cpu(g.text().replace("@hip:0", "@cpu:0"), [a, gy])
    assert_bitwise(out.numpy(), want, "eager matmul_grad_rhs")


# ---- conv gradients ------------------------------------------------------------------------------------------

CONV_CASES = [
    # (N, Cin, H, W, Cout, K, stride, pad, groups); Cout % 32 == 0 (16-bit) / % 16 (fp32): grad_input runs as a
    # transposed convolution on the implicit-GEMM kernel (tolerance), otherwise on the direct kernel (bit-exact)
    (2, 32, 9, 9, 64, 3, 1, 1, 1),
    (2, 64, 10, 11, 128, 3, 2, 1, 1),
    (2, 16, 9, 9, 160, 3, 1, 1, 1),   # Cout >= 128 with a partial 128-row filter-gradient tile
    (2, 64, 10, 10, 128, 1, 2, 0, 1),
    (2, 16, 15, 15, 64, 7, 2, 3, 1),
    (2, 3, 20, 20, 64, 7, 2, 3, 1),
    (4, 64, 14, 14, 64, 3, 1, 1, 1),
    (2, 8, 9, 9, 16, 3, 1, 1, 1),
    (2, 8, 9, 10, 16, 3, 2, 1, 1),
    (3, 16, 8, 8, 8, 1, 2, 0, 1),
    (2, 3, 15, 15, 8, 7, 2, 3, 1),
    (2, 8, 6, 6, 8, 3, 1, 0, 2),
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", CONV_CASES)
def test_conv_grads(dev, dtype, case):
    n, cin, h, w, cout, kk, s, p, grp = case
    say(f"conv grads {case} dtype={dtype}")
    oh, ow = conv_out(h, kk, s, p), conv_out(w, kk, s, p)
    xs, ws, dys = (n, cin, h, w), (cout, cin // grp, kk, kk), (n, cout, oh, ow)
    x, wt, dy = tensors(40, [xs, ws, dys], dtype)
    common = {"stride": [s, s], "padding": [p, p], "groups": grp}
    gi = one_op("conv2d_grad_input_internal", [dys, ws], xs, dict(common, input_shape=graphs.Shape(xs)), dtype)
    got, want = both(gi, [dy, wt])
    if "hip_conv2d_nhwc_internal" in host.hip_lowered(gi.text()):
        assert_close(got[0], want[0], dtype, what="conv2d_grad_input (implicit GEMM)")
    else:
        assert_bitwise(got[0], want[0], "conv2d_grad_input")
    gf = one_op("conv2d_grad_filter_internal", [xs, dys], ws, dict(common, filter_shape=graphs.Shape(ws)), dtype)
    got, want = both(gf, [x, dy])
    if "hip_conv2d_wgrad_nhwc_internal" in host.hip_lowered(gf.text()):
        assert_close(got[0], want[0], dtype, what="conv2d_grad_filter (MFMA, split-K)")
    else:
        assert_bitwise(got[0], want[0], "conv2d_grad_filter")


# ---- pool gradients ------------------------------------------------------------------------------------------

POOL_CASES = [
    # (N, C, H, W, K, stride, pad)
    (2, 4, 17, 16, 3, 2, 1),
    (2, 3, 8, 8, 2, 2, 0),
    (1, 5, 7, 7, 7, 7, 0),
    (2, 2, 9, 9, 3, 1, 1),
    (2, 8, 24, 32, 3, 2, 1),  # 3x3/s2/p1 with W % 8 == 0: the 2x8-block kernel, planes staged in LDS
    (2, 4, 18, 24, 3, 2, 1),  # ... with a dy plane (9 x 12) that is not whole 16-byte vectors
    (2, 3, 112, 112, 3, 2, 1),  # ResNet's stem pool plane
    (1, 2, 192, 192, 3, 2, 1),  # planes too large for LDS: the per-thread 2x8-block kernel
    (1, 3, 13, 13, 3, 2, 1),  # ... and the 2x2-block kernel
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", POOL_CASES)
def test_pool_grads(dev, dtype, case):
    n, c, h, w, kk, s, p = case
    say(f"pool grads {case} dtype={dtype}")
    oh, ow = conv_out(h, kk, s, p), conv_out(w, kk, s, p)
    xs, dys = (n, c, h, w), (n, c, oh, ow)
    x, dy = tensors(50, [xs, dys], dtype)
    x.reshape(-1)[::7] = x.reshape(-1)[3]  # repeated values: ties resolve to the first maximum
    attrs = {"kernel": [kk, kk], "stride": [s, s], "padding": [p, p], "input_shape": graphs.Shape(xs)}
    got, want = both(one_op("max_pool2d_grad_internal", [dys, xs], xs, attrs, dtype), [dy, x])
    assert_bitwise(got[0], want[0], "max_pool2d_grad")
    got, want = both(one_op("avg_pool2d_grad_internal", [dys], xs, attrs, dtype), [dy])
    assert_bitwise(got[0], want[0], "avg_pool2d_grad")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(2, 64, 9, 9), (3, 1000, 17), (5, 7)])
def test_masked_gradient_sum(dev, dtype, shape):
    """relu_grad_internal(x, add(a, b)) lowers to one add-then-mask program (FH_EW_RELU_MASK) on hip; the oracle
    runs the add and the relu_grad. x holds zeros and negatives; odd sizes take the element tail."""
    say(f"masked gradient sum {shape} dtype={dtype}")
    a, b, x = tensors(70, [shape, shape, shape], dtype)
    x.reshape(-1)[::4] = 0
    g = graphs.Graph("hip")
    va, vb, vx = g.input(dtype, shape), g.input(dtype, shape), g.input(dtype, shape)
    g.output(g.op("relu_grad_internal", [vx, g.add(va, vb)], shape, {}))
    assert "ew_ops=[1, 11]" in host.hip_lowered(g.text(), 1)
    got, want = both(g, [a, b, x])
    assert_bitwise(got[0], want[0], "masked gradient sum")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", [c for c in POOL_CASES if c[4] == 3])
def test_max_pool_relu_grad(dev, dtype, case):
    """relu_grad_internal(x, max_pool2d_grad_internal(dy, x)) lowers to one fused launch (fh_pool2d_grad mode 2)
    on hip; the oracle runs the two ops. x holds negatives, zeros and ties."""
    n, c, h, w, kk, s, p = case
    say(f"max_pool relu grad {case} dtype={dtype}")
    oh, ow = conv_out(h, kk, s, p), conv_out(w, kk, s, p)
    xs, dys = (n, c, h, w), (n, c, oh, ow)
    x, dy = tensors(60, [xs, dys], dtype)
    x.reshape(-1)[::7] = x.reshape(-1)[3]
    x.reshape(-1)[::5] = 0
    attrs = {"kernel": [kk, kk], "stride": [s, s], "padding": [p, p], "input_shape": graphs.Shape(xs)}
    g = graphs.Graph("hip")
    vdy, vx = g.input(dtype, dys), g.input(dtype, xs)
    m = g.op("max_pool2d_grad_internal", [vdy, vx], xs, attrs)
    g.output(g.op("relu_grad_internal", [vx, m], xs, {}))
    assert "hip_max_pool2d_relu_grad_internal" in host.hip_lowered(g.text(), 1)
    got, want = both(g, [dy, x])
    assert_bitwise(got[0], want[0], "max_pool2d relu grad")


# ---- sum, sum_grad, mse_loss -----------------------------------------------------------------------------------

SUM_CASES = [((4, 6, 5, 7), [0, 2, 3], False), ((4, 6, 5, 7), [], False), ((33, 1000), [1], True),
             ((33, 1000), [0], False), ((8, 3, 300), [0, 2], False), ((1 << 20,), [], False),
             ((8, 64, 28, 28), [0, 2, 3], False), ((3, 5, 9, 9), [0, 2, 3], True),
             # every axis but the last, >= 256 rows: the two-pass column sum (hip_sum_rows_internal)
             ((5000, 64), [0], False), ((4096, 24), [0], False), ((300, 8, 8), [0, 1], False)]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape,axes,keep", SUM_CASES)
def test_sum_and_sum_grad(dev, dtype, shape, axes, keep):
    say(f"sum {shape} axes={axes} keepdims={keep} dtype={dtype}")
    red = set(range(len(shape))) if not axes else set(axes)
    out = tuple((1 if keep else None) if i in red else d for i, d in enumerate(shape))
    out = tuple(d for d in out if d is not None)
    attrs = {"axes": list(axes)}
    if keep:
        attrs["keepdims"] = True
    (x,) = tensors(60, [shape], dtype)
    got, want = both(one_op("sum", [shape], out, attrs, dtype), [x])
    # fp32 tree vs the reference's sequential sum: bound by the sum of magnitudes
    mag = np.abs(x.astype(np.float32) if dtype == F32 else synth.to_float(x, dtype)).sum(
        axis=tuple(sorted(red)), keepdims=keep).reshape(out)
    g32 = got[0] if dtype == F32 else synth.to_float(got[0], dtype)
    w32 = want[0] if dtype == F32 else synth.to_float(want[0], dtype)
    tol = (2e-6 * mag) if dtype == F32 else (1e-2 * np.abs(w32) + 1e-5 * mag)
    assert np.all(np.abs(g32 - w32) <= tol), f"sum: max excess {np.max(np.abs(g32 - w32) - tol)}"
    (gy,) = tensors(61, [out], dtype)
    gattrs = {"axes": list(axes), "input_shape": graphs.Shape(shape)}
    got, want = both(one_op("sum_grad_internal", [out], shape, gattrs, dtype), [gy])
    assert_bitwise(got[0], want[0], "sum_grad")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(64, 10), (1000, 513), (7,)])
def test_mse_loss_and_grad(dev, dtype, shape):
    say(f"mse_loss {shape} dtype={dtype}")
    p, t = tensors(70, [shape, shape], dtype)
    got, want = both(one_op("mse_loss", [shape, shape], (), None, dtype), [p, t])
    # The reference sums sequentially in fp32 (its error grows with numel: 1.7e-4 relative at 513k terms); the
    # kernel's tree is checked against the float64 value of the same storage inputs, and must be at least as close
    # to it as the reference is, up to the tolerance.
    truth = float(np.mean((synth.to_float(p, dtype).astype(np.float64) - synth.to_float(t, dtype).astype(np.float64)) ** 2))
    g = float(synth.to_float(np.asarray(got[0]).reshape(1), dtype)[0])
    w = float(synth.to_float(np.asarray(want[0]).reshape(1), dtype)[0])
    rtol = {F32: 1e-5, BF16: 8e-3, F16: 1e-3}[dtype]
    assert abs(g - truth) <= rtol * truth, (g, truth)
    assert abs(g - w) <= abs(w - truth) + rtol * truth, (g, w, truth)
    (gy,) = tensors(72, [()], dtype)
    got, want = both(one_op("mse_loss_grad_internal", [shape, shape, ()], shape, None, dtype), [p, t, gy])
    assert_bitwise(got[0], want[0], "mse_loss_grad")


# ---- whole training graphs -----------------------------------------------------------------------------------

def check_outputs(got, want, dtype, what):
    assert len(got) == len(want)
    for i, (a, b) in enumerate(zip(got, want)):
        assert_close(np.asarray(a).reshape(-1), np.asarray(b).reshape(-1), dtype, what=f"{what} output {i}")


@pytest.mark.parametrize("dtype", [F32, BF16])
def test_mlp_training_step(dev, dtype):
    # C1's MLP under mse_loss: loss, d/dw1, d/db1, d/dw2, d/db2
    say(f"mlp training step dtype={dtype}")
    g = graphs.mlp_train(batch=64, dtype=dtype, device="hip")
    text = host.backward(g.text(), 0, [1, 2, 3, 4])
    ins = graphs.mlp_train_inputs(batch=64, dtype=dtype)
    got = host.compile(text, "hip", 1).run(ins)
    want = orc.run_graph_cpu(text.replace("@hip:0", "@cpu:0"), ins)
    check_outputs(got, want, dtype, "mlp training")
    if dtype == F32:
        # at opt_level 0 every GEMM below the tiled threshold keeps the reference's order: the gradients are
        # bit-exact (opt_level 1 lets the forward's fused small GEMMs reassociate k, checked within tolerance above)
        got0 = host.compile(text, "hip", 0).run(ins)
        for i in range(1, 5):
            assert_bitwise(got0[i], want[i], f"mlp gradient {i} at opt_level 0")


@pytest.mark.parametrize("dtype", [F32, BF16])
def test_cnn_training_step(dev, dtype):
    say(f"cnn training step dtype={dtype}")
    g = graphs.cnn_train(batch=4, dtype=dtype, device="hip")
    text = host.backward(g.text(), 0, [1, 2, 3, 4, 5, 6])
    ins = graphs.cnn_train_inputs(batch=4, dtype=dtype)
    got = host.compile(text, "hip", 1).run(ins)
    want = orc.run_graph_cpu(text.replace("@hip:0", "@cpu:0"), ins)
    check_outputs(got, want, dtype, "cnn training")


@pytest.mark.parametrize("dtype", [F32, BF16])
def test_sgd_update(dev, dtype):
    say(f"sgd update dtype={dtype}")
    g = graphs.mlp_train(batch=64, dtype=dtype, device="hip")
    text = host.sgd_update(g.text(), [1, 2, 3, 4], 0.05)
    params = graphs.mlp_train_inputs(batch=64, dtype=dtype)[1:5]
    grads = [synth.tensor(80 + i, p.shape, dtype) for i, p in enumerate(params)]
    got = host.compile(text, "hip", 1).run(params + grads)
    want = orc.run_graph_cpu(text.replace("@hip:0", "@cpu:0"), params + grads)
    for i in range(4):
        assert_bitwise(got[i], want[i], f"sgd param {i}")


@pytest.mark.parametrize("dtype", [F32, BF16])
@pytest.mark.parametrize("act", ["gelu", "relu"])
def test_transformer_training_step(dev, dtype, act):
    # C5's block at a small size: gradients of layer_norm, softmax, slice / concat / transpose, gelu or relu
    say(f"transformer training step act={act} dtype={dtype}")
    shape = dict(batch=2, seq=64, d_model=128, heads=2, ffn=256)
    g, shapes = graphs.transformer_block(dtype=dtype, act=act, train=True, **shape)
    text = host.backward(g.text(), 0, list(range(1, len(shapes) + 1)))
    rows = shape["batch"] * shape["seq"]
    ins = graphs.transformer_inputs(shapes, rows=rows, d_model=128, dtype=dtype) + [synth.tensor(77, (rows, 128), dtype)]
    got = host.compile(text, "hip", 1).run(ins)
    want = orc.run_graph_cpu(text.replace("@hip:0", "@cpu:0"), ins)
    check_outputs(got, want, dtype, f"transformer training ({act})")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("op", ["sigmoid", "tanh", "rsqrt"])
def test_unary_ops(dev, dtype, op):
    say(f"{op} dtype={dtype}")
    shape = (37, 129)
    (x,) = tensors(90, [shape], dtype)
    if op == "rsqrt":
        x = synth.to_storage(np.abs(synth.to_float(x, dtype)) + 0.05, dtype)
    got, want = both(one_op(op, [shape], shape, None, dtype), [x])
    if op == "rsqrt" or dtype != F32:
        assert_bitwise(got[0], want[0], op)  # correctly rounded sqrt / divide; 16-bit rounding absorbs the rest
    else:
        assert_close(got[0], want[0], dtype, what=op)  # device expf / tanhf vs the C library: a few ulp


@pytest.mark.parametrize("dtype", DTYPES)
def test_gelu_grad(dev, dtype):
    say(f"gelu_grad dtype={dtype}")
    shape = (64, 513)
    x, gy = tensors(95, [shape, shape], dtype)
    got, want = both(one_op("gelu_grad_internal", [shape, shape], shape, None, dtype), [x, gy])
    assert_close(got[0], want[0], dtype, what="gelu_grad")


@pytest.mark.parametrize("dtype", DTYPES)
def test_sgd_update_many_params(dev, dtype):
    # 40 parameters (two multi-tensor launches of 32 + 8 pairs), sizes with ragged 16-byte tails and one element
    say(f"sgd update 40 params dtype={dtype}")
    shapes = [(1,), (13,), (8,), (1000,), (64, 3, 7, 7), (4099,), (7, 9), (512, 512, 3, 3)] * 5
    g = graphs.Graph("hip")
    vals = [g.input(dtype, s) for s in shapes]
    g.output(g.op("relu", [vals[0]], shapes[0]))
    text = host.sgd_update(g.text(), list(range(len(shapes))), 0.03)
    assert host.hip_lowered(text).count("hip_axpy_multi_internal(") == 2
    params = [synth.tensor(200 + i, s, dtype).reshape(s) for i, s in enumerate(shapes)]
    grads = [synth.tensor(300 + i, s, dtype).reshape(s) for i, s in enumerate(shapes)]
    got = host.compile(text, "hip", 1).run(params + grads)
    want = orc.run_graph_cpu(text.replace("@hip:0", "@cpu:0"), params + grads)
    for i in range(len(shapes)):
        assert_bitwise(got[i], want[i], f"sgd param {i} {shapes[i]}")


def test_axpy_multi_unaligned(dev):
    # fh_axpy_multi directly: tensors starting 4 bytes into their buffers take the element path
    from frame_hip import abi
    import ctypes
    say("axpy_multi unaligned f32")
    rng = np.random.default_rng(9)
    sizes, scales = [37, 1024, 5], [-0.5, 0.25, 3.0]
    xs = [rng.standard_normal(n + 1).astype(np.float32) for n in sizes]
    ys = [rng.standard_normal(n + 1).astype(np.float32) for n in sizes]
    dx = [host.Tensor.from_numpy("hip", F32, a) for a in xs]
    dy = [host.Tensor.from_numpy("hip", F32, a) for a in ys]
    do = [host.Tensor("hip", F32, (n + 1,)) for n in sizes]
    off = [0, 1, 1]  # tensor 0 aligned, tensors 1 and 2 shifted by one element
    k = len(sizes)
    P = ctypes.c_void_p * k
    xp = P(*[t.data_ptr + 4 * o for t, o in zip(dx, off)])
    yp = P(*[t.data_ptr + 4 * o for t, o in zip(dy, off)])
    op = P(*[t.data_ptr + 4 * o for t, o in zip(do, off)])
    abi.check(abi.lib().fh_axpy_multi(F32, k, xp, yp, op, (ctypes.c_int64 * k)(*sizes), (ctypes.c_float * k)(*scales), None))
    abi.check(abi.lib().fh_device_synchronize())
    for i, n in enumerate(sizes):
        o = off[i]
        want = xs[i][o:o + n] + (np.float32(scales[i]) * ys[i][o:o + n])
        assert_bitwise(do[i].numpy()[o:o + n], want, f"axpy tensor {i}")

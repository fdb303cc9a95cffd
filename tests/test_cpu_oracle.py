"""The parity oracle (oracle/cpu_kernels.cpp and its `cpu` backend) pinned on the CPU:
  * against the reference built from its own sources (oracle/_ref), bit for bit, on the hot-path ops;
  * against the known answers of the reference's own op tests;
  * against closed forms that a plausible slip (dropped term, wrong index, transposed operand, missing bias,
    wrong rounding point) would break: fp64 recomputation, im2col, invariants and exhaustive dtype sweeps.
"""
import ctypes
import math

import numpy as np
import pytest

import oracle_lib as orc
from frame_hip import graphs, synth
from tolerance import assert_bitwise

F32, F16, BF16 = 0, 2, 3
needs_ref = pytest.mark.skipif(not orc.ref_available(), reason="oracle/_ref not built (no /root/reference here)")


def ref_graph(g, ins):
    """The same graph text on the reference's own CPU backend."""
    specs = []
    for v in g.outputs:
        specs.append((v.shape, np.float32 if v.dtype == F32 else np.uint16))
    return orc.ref_run_graph(g.text(), ins, specs)


# ---- dtype bridge -------------------------------------------------------------------------------------------

def test_widening_exhaustive_closed_form():
    o = orc.oracle()
    for code, fn, to_f in ((BF16, o.oracle_bf16_to_float, synth.bf16_bits_to_f32),
                           (F16, o.oracle_f16_to_float, synth.f16_bits_to_f32)):
        bits = np.arange(65536, dtype=np.uint16)
        want = to_f(bits)  # numpy: bf16 = upper half of float32; f16 = IEEE binary16 widening
        got = np.array([fn(int(b)) for b in bits[::97]], dtype=np.float32)
        w = want[::97]
        same = (got.view(np.uint32) == w.view(np.uint32)) | (np.isnan(got) & np.isnan(w))
        assert same.all(), code


def test_narrowing_against_numpy_sample():
    # float16: numpy's IEEE round-to-nearest-even cast; bfloat16: the textbook bias-and-truncate rule
    rng = np.random.default_rng(0)
    u = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    specials = np.array([0, 0x80000000, 0x7f800000, 0xff800000, 0x7fc00001, 0x33000000, 0x33000001, 0x387fc000,
                         0x477fefff, 0x477ff000, 0x3f808000, 0x3f818000], np.uint32)
    u = np.concatenate([u, specials])
    f = u.view(np.float32)
    out16 = np.empty(len(f), np.uint16)
    orc.oracle().oracle_f32_to_f16_array(f.ctypes.data, out16.ctypes.data, len(f))
    assert_bitwise(out16, synth.f32_to_f16_bits(f), "f16 narrowing")
    outb = np.empty(len(f), np.uint16)
    orc.oracle().oracle_f32_to_bf16_array(f.ctypes.data, outb.ctypes.data, len(f))
    assert_bitwise(outb, synth.f32_to_bf16_bits(f), "bf16 narrowing")


@needs_ref
def test_narrowing_exhaustive_against_reference():
    # all 2^32 float32 patterns through both narrowings, compared with the reference's dtype.h functions
    o = orc.oracle()
    proto = ctypes.CFUNCTYPE(ctypes.c_uint16, ctypes.c_float)
    bf = ctypes.cast(o.oracle_float_to_bf16, ctypes.c_void_p)
    hf = ctypes.cast(o.oracle_float_to_f16, ctypes.c_void_p)
    first = ctypes.c_uint32(0)
    bad = orc.ref().ref_compare_narrowing_exhaustive(bf, hf, ctypes.byref(first))
    assert bad == 0, f"{bad} mismatches, first input bits {first.value:#010x}"
    del proto


# ---- known answers from the reference's op tests -------------------------------------------------------------

def test_matmul_known_answer():
    # reference: tests/cpp/ops/test_op_matmul.cpp:208-230
    a = np.array([[1, 2], [3, 4]], np.float32)
    b = np.array([[5, 6], [7, 8]], np.float32)
    assert_bitwise(orc.matmul(F32, a, b), np.array([[19, 22], [43, 50]], np.float32), "matmul")


def test_softmax_known_answer():
    # reference: tests/cpp/ops/test_op_softmax.cpp:123-162
    y = orc.softmax(F32, np.array([[1, 2], [3, 4]], np.float32))
    np.testing.assert_allclose(y, [[0.26894142, 0.73105858]] * 2, rtol=1e-6)


def test_layer_norm_known_answer():
    # reference: tests/cpp/ops/test_op_layer_norm.cpp:230-253 (eps = 1e-5)
    x = np.array([[1, 2, 3, 4], [0, 2, 4, 6]], np.float32)
    g = np.array([2.0, 0.5, 1.0, -1.0], np.float32)
    b = np.array([0.1, -0.2, 0.0, 1.0], np.float32)
    want = [[-2.5832708, -0.4236059, 0.4472118, -0.3416354], [-2.5832789, -0.4236066, 0.4472131, -0.3416394]]
    np.testing.assert_allclose(orc.layer_norm(F32, x, g, b, 1e-5), want, rtol=1e-5, atol=1e-6)


def test_gelu_known_points():
    # gelu(x) = 0.5 x (1 + erf(x / sqrt 2)): gelu(0) = 0, gelu(1) = 0.8413447, gelu(-1) = -0.1586553, tails
    x = np.array([0.0, 1.0, -1.0, 10.0, -10.0, 3.0], np.float32)
    y = orc.ew_program(F32, [5], [1], [x])
    want = [0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x.astype(np.float64)]
    np.testing.assert_allclose(y, want, rtol=2e-7, atol=1e-7)
    assert y[0] == 0.0 and abs(y[4]) < 1e-20


def test_relu_special_values():
    # relu is std::max(x, 0.0f): NaN and -0.0 pass through (reference: src/backends/cpu/kernels/elementwise.cpp:323-330)
    x = np.array([np.nan, -0.0, 0.0, -1.5, 2.5, np.inf, -np.inf], np.float32)
    y = orc.ew_program(F32, [3], [1], [x])
    assert np.isnan(y[0]) and np.signbit(y[1]) and y[3] == 0.0 and y[5] == np.inf and y[6] == 0.0


# ---- closed forms -----------------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [F32, BF16])
def test_matmul_against_fp64(dtype):
    a = synth.tensor(3, (37, 129), dtype, "uniform")
    b = synth.tensor(4, (129, 53), dtype, "uniform")
    got = synth.to_float(orc.matmul(dtype, a, b), dtype).astype(np.float64)
    want = synth.to_float(a, dtype).astype(np.float64) @ synth.to_float(b, dtype).astype(np.float64)
    bound = 129 * 2**-23 * (np.abs(synth.to_float(a, dtype)) @ np.abs(synth.to_float(b, dtype))) + (
        np.abs(want) * (2**-8 if dtype == BF16 else 0))
    assert np.all(np.abs(got - want) <= bound + 1e-30)


def test_matmul_sample_equals_full():
    a = synth.tensor(5, (31, 70), BF16, "uniform")
    b = synth.tensor(6, (70, 45), BF16, "uniform")
    full = orc.matmul(BF16, a, b)
    rows, cols = np.array([0, 30, 7, 12]), np.array([44, 0, 9, 33])
    assert_bitwise(orc.matmul_sample(BF16, a, b, rows, cols), full[rows, cols], "sample")


@pytest.mark.parametrize("geom", [(2, 3, 9, 9, 4, 7, 7, 2, 2, 3, 3, 1), (1, 4, 6, 5, 6, 3, 3, 1, 1, 1, 1, 2)])
def test_conv_against_im2col(geom):
    n, cin, h, w, cout, kh, kw, sh, sw, ph, pw, groups = geom
    x = synth.tensor(7, (n, cin, h, w), F32, "normal")
    wt = synth.tensor(8, (cout, cin // groups, kh, kw), F32, "normal")
    bias = synth.tensor(9, (cout,), F32, "normal")
    got = orc.conv2d(F32, x, wt, bias, geom).astype(np.float64)
    oh, ow = orc.conv_out_hw(geom)
    xp = np.pad(x.astype(np.float64), ((0, 0), (0, 0), (ph, ph), (pw, pw)))
    want = np.zeros((n, cout, oh, ow))
    cg, og = cin // groups, cout // groups
    for co in range(cout):
        grp = co // og
        for i in range(oh):
            for j in range(ow):
                patch = xp[:, grp * cg:(grp + 1) * cg, i * sh:i * sh + kh, j * sw:j * sw + kw]
                want[:, co, i, j] = (patch * wt[co].astype(np.float64)).reshape(n, -1).sum(1) + bias[co]
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_softmax_invariants():
    x = synth.tensor(10, (6, 300), F32, "normal", 3.0)
    y = orc.softmax(F32, x).astype(np.float64)
    np.testing.assert_allclose(y.sum(1), 1.0, rtol=1e-5)
    y2 = orc.softmax(F32, (x + np.float32(7.0))).astype(np.float64)  # shift invariance
    np.testing.assert_allclose(y, y2, rtol=1e-5, atol=1e-8)
    ref = np.exp(x - x.max(1, keepdims=True)).astype(np.float64)
    np.testing.assert_allclose(y, ref / ref.sum(1, keepdims=True), rtol=2e-6, atol=1e-9)


def test_layer_norm_closed_form():
    x = synth.tensor(11, (5, 257), F32, "normal", 2.0)
    g = synth.tensor(12, (257,), F32, "normal")
    b = synth.tensor(13, (257,), F32, "normal")
    y = orc.layer_norm(F32, x, g, b, 1e-5).astype(np.float64)
    xd = x.astype(np.float64)
    want = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-5) * g + b
    np.testing.assert_allclose(y, want, rtol=1e-4, atol=1e-5)


def test_pool_brute_force():
    x = synth.tensor(14, (2, 3, 7, 8), F32, "normal")
    geom = (2, 3, 7, 8, 3, 3, 2, 2, 1, 1)
    got = orc.pool2d(F32, 0, x, geom)
    xp = np.pad(x, ((0, 0), (0, 0), (1, 1), (1, 1)), constant_values=-np.inf)
    want = np.zeros_like(got)
    for i in range(got.shape[2]):
        for j in range(got.shape[3]):
            want[:, :, i, j] = xp[:, :, 2 * i:2 * i + 3, 2 * j:2 * j + 3].max(axis=(2, 3))
    assert_bitwise(got, want, "max pool")
    gavg = orc.pool2d(F32, 1, x, geom).astype(np.float64)
    xz = np.pad(x.astype(np.float64), ((0, 0), (0, 0), (1, 1), (1, 1)))
    wavg = np.zeros_like(gavg)
    for i in range(gavg.shape[2]):
        for j in range(gavg.shape[3]):
            wavg[:, :, i, j] = xz[:, :, 2 * i:2 * i + 3, 2 * j:2 * j + 3].sum(axis=(2, 3)) / 9.0
    np.testing.assert_allclose(gavg, wavg, rtol=1e-6, atol=1e-7)


def test_fused_program_equals_unfused_sequence():
    # one program == the same ops one by one with a rounding after each (reference: fused_elementwise_utils.cpp:122-206)
    x, y, z = (synth.tensor(s, (4096,), BF16, "normal") for s in (15, 16, 17))
    fused = orc.ew_program(BF16, [1, 2, 3], [2, 2, 1], [x, y, z])
    step = orc.ew_program(BF16, [1], [2], [x, y])
    step = orc.ew_program(BF16, [2], [2], [step, z])
    step = orc.ew_program(BF16, [3], [1], [step])
    assert_bitwise(fused, step, "fused vs unfused")


# ---- whole graphs: oracle `cpu` backend vs the reference's cpu backend, bit for bit -----------------------------

@needs_ref
@pytest.mark.parametrize("dtype", [F32, BF16])
def test_mlp_graph_bitexact_vs_reference(dtype):
    g = graphs.mlp(batch=16, dtype=dtype, device="cpu")
    ins = graphs.mlp_inputs(batch=16, dtype=dtype, seed=3)
    (mine,) = orc.run_graph_cpu(g, ins)
    (ref,) = ref_graph(g, ins)
    assert_bitwise(mine, ref, "mlp")


@needs_ref
@pytest.mark.parametrize("dtype", [F32, BF16])
@pytest.mark.parametrize("shape", [(64, 576, 64), (17, 4096, 3), (5, 7, 9)])
def test_matmul_graph_bitexact_vs_reference(dtype, shape):
    m, k, n = shape
    g = graphs.gemm(n, dtype, device="cpu", m=m, k=k)
    ins = graphs.gemm_inputs(n, dtype, m=m, k=k)
    assert_bitwise(orc.run_graph_cpu(g, ins)[0], ref_graph(g, ins)[0], f"matmul {shape}")


@needs_ref
@pytest.mark.parametrize("dtype", [F32, BF16])
@pytest.mark.parametrize("cfg", [dict(n=2, cin=3, h=9, w=9, cout=4, k=7, stride=2, pad=3),
                                 dict(n=2, cin=8, h=7, w=7, cout=8, k=3, stride=1, pad=1),
                                 dict(n=1, cin=16, h=14, w=14, cout=32, k=1, stride=2, pad=0)])
def test_conv_graph_bitexact_vs_reference(dtype, cfg):
    g = graphs.conv(dtype, device="cpu", **cfg)
    ins = graphs.conv_inputs(dtype, n=cfg["n"], cin=cfg["cin"], h=cfg["h"], w=cfg["w"], cout=cfg["cout"], k=cfg["k"])
    assert_bitwise(orc.run_graph_cpu(g, ins)[0], ref_graph(g, ins)[0], f"conv {cfg}")


@needs_ref
def test_resnet_tiny_bitexact_vs_reference():
    g, specs = graphs.resnet18(batch=1, dtype=BF16, device="cpu", image=32, classes=10)
    ins = graphs.resnet18_inputs(specs, batch=1, dtype=BF16, image=32)
    assert_bitwise(orc.run_graph_cpu(g, ins)[0], ref_graph(g, ins)[0], "resnet18 32px")


def _tiny_block(device, act="gelu"):
    g, shapes = graphs.transformer_block(batch=2, seq=16, d_model=32, heads=2, ffn=64, dtype=BF16, device=device)
    text = g.text()
    if act != "gelu":
        text = text.replace(" gelu(", f" {act}(")
    return g, shapes, text


@needs_ref
def test_transformer_tiny_bitexact_vs_reference():
    # The reference has no gelu op: the relu variant of the same block is compared with the reference.
    g, shapes, text = _tiny_block("cpu", act="relu")
    ins = graphs.transformer_inputs(shapes, rows=32, d_model=32, dtype=BF16)
    (mine,) = orc.run_graph_cpu(text, ins)
    (ref,) = orc.ref_run_graph(text, ins, [((32, 32), np.uint16)])
    assert_bitwise(mine, ref, "transformer (relu) tiny")

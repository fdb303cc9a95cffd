"""The drop-in proof on the MI355X: the reference's OWN runtime drives the hip plugin. oracle/_ref/libframe_dropin.so
links the reference's sources (runtime::compile with its cache, the nine-pass pipeline, backend_lowering and
FallbackExecutable, run_with_allocated_outputs, the cpu backend) with this repository's plugin sources compiled
unchanged against the reference's headers (tests/dropin_lib.py, oracle/Makefile target dropin). Every graph is
compiled by the reference's runtime::compile(graph, "hip") and run by its run_with_allocated_outputs, and checked
against the same graph on the reference's own cpu backend in the same library (rtol 1e-5 float32, 1e-2
bfloat16, atol = rtol * rms(expected), tests/tolerance.py; data movement and elementwise ops bit for bit).

The reference's CUDA backend behaviour cases are mirrored for hip (reference
tests/cpp/backends/test_cuda_backend.cpp): end-to-end compile with a second compile served by the cache and no
FallbackStats entries (:1579-1655), the cross-device fallback sandwich (:1663-1737), cpu tensors refused with a
message naming both backends (:1744-1767), empty add/mul graphs (:2201-2205) and the vectorization boundary at
numel 1023/1024 for add and relu in float32, float16 and bfloat16 (:1252-1290).
"""
import numpy as np
import pytest

import dropin_lib as dl
from frame_hip import graphs, synth
from tolerance import assert_bitwise, assert_close

pytestmark = pytest.mark.gpu
F32, F16, BF16 = 0, 2, 3


def say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def dev():
    assert dl.available(), "oracle/_ref/libframe_dropin.so missing: build it where the reference tree exists"
    assert "hip" in dl.backends()
    n = dl.device_count("hip")
    assert n >= 1, "no hip device visible to the reference runtime"
    return n


def on_cpu(text):
    return text.replace("@hip:0", "@cpu:0")


def both(text, ins, opt_level=1):
    got = dl.Executable(text, "hip", opt_level).run(ins)
    want = dl.Executable(on_cpu(text), "cpu").run(ins)
    assert len(got) == len(want)
    return got, want


@pytest.mark.parametrize("opt_level", [0, 1])
def test_c1_mlp_through_the_reference_runtime(dev, opt_level):
    say(f"drop-in C1 batch 64 f32 opt_level {opt_level}")
    text = graphs.mlp(batch=64, dtype=F32, device="hip").text()
    (got,), (want,) = both(text, graphs.mlp_inputs(batch=64, dtype=F32), opt_level)
    assert_close(got, want, F32, what="C1 via reference runtime")


@pytest.mark.parametrize("dtype", [F32, BF16])
def test_c3_conv_through_the_reference_runtime(dev, dtype):
    for cfg in (dict(n=2, cin=64, h=16, w=16, cout=64, k=3), dict(n=2, cin=3, h=20, w=20, cout=16, k=7, stride=2, pad=3)):
        say(f"drop-in C3 {cfg} dtype {dtype}")
        text = graphs.conv(dtype, device="hip", **cfg).text()
        ins = graphs.conv_inputs(dtype, n=cfg["n"], cin=cfg["cin"], h=cfg["h"], w=cfg["w"], cout=cfg["cout"], k=cfg["k"])
        (got,), (want,) = both(text, ins)
        assert_close(got, want, dtype, what=f"C3 {cfg} via reference runtime")


def test_c5_small_through_the_reference_runtime(dev):
    say("drop-in C5 small (relu FFN) bf16")
    g, shapes = graphs.transformer_block(batch=2, seq=128, d_model=256, heads=4, ffn=512, dtype=BF16, act="relu")
    ins = graphs.transformer_inputs(shapes, rows=256, d_model=256, dtype=BF16)
    (got,), (want,) = both(g.text(), ins)
    assert_close(got, want, BF16, what="C5 small via reference runtime")


def test_second_compile_hits_the_cache_and_nothing_falls_back(dev):
    say("drop-in compile cache and FallbackStats")
    g = graphs.Graph("hip")
    x, w, b = g.input(F32, (2, 3)), g.input(F32, (3, 4)), g.input(F32, (2, 4))
    g.output(g.relu(g.add(g.matmul(x, w), b)))
    first, second = dl.Executable(g.text(), "hip"), dl.Executable(g.text(), "hip")
    assert first.identity() == second.identity() != 0
    ins = [np.array([[1, 2, 3], [4, 5, 6]], np.float32),
           np.array([[0.1, -0.2, 0.3, -0.4], [0.5, -0.6, 0.7, -0.8], [0.9, -1.0, 1.1, -1.2]], np.float32),
           np.array([[0.25, -0.5, 0.75, -1.0], [-0.25, 0.5, -0.75, 1.0]], np.float32)]
    (r1,), (r2,) = first.run(ins), second.run(ins)
    (want,) = dl.Executable(on_cpu(g.text()), "cpu").run(ins)
    assert_close(r1, want, F32, what="matmul;add;relu")
    assert_bitwise(r2, r1, "second executable")
    for op in ("matmul", "add", "relu", "fused_elementwise_internal"):
        assert dl.fallback_count(op, "hip") == 0, op


def test_cross_device_fallback_sandwich(dev):
    """add (hip) -> an op with only a cpu kernel -> relu (hip): the reference's backend_lowering sends the graph to
    FallbackExecutable, which launches add and relu through HipBackend::launch and copies around the cpu op."""
    say("drop-in fallback sandwich")
    op = dl.sandwich_op()
    g = graphs.Graph("hip")
    a, b = g.input(F32, (4,)), g.input(F32, (4,))
    g.output(g.relu(g.op(op, [g.add(a, b)], (4,))))
    before = dl.fallback_count(op, "hip")
    ins = [np.array([1.0, -2.0, 3.0, 0.5], np.float32), np.array([2.0, 1.0, -4.0, 0.5], np.float32)]
    (got,), (want,) = both(g.text(), ins)
    assert_bitwise(got, want, "sandwich vs cpu")
    assert_bitwise(got, np.maximum(2.0 * (ins[0] + ins[1]) - 1.0, 0.0).astype(np.float32), "sandwich closed form")
    assert dl.fallback_count(op, "hip") == before + 1
    assert dl.fallback_count("add", "hip") == 0 and dl.fallback_count("relu", "hip") == 0


def test_run_refuses_cpu_tensors_naming_both_backends(dev):
    say("drop-in device check")
    g = graphs.Graph("hip")
    x = g.input(F32, (4,))
    g.output(g.relu(x))
    rc, msg = dl.Executable(g.text(), "hip").run_with_host_inputs([np.array([1, -1, 2, -2], np.float32)])
    assert rc == 1, (rc, msg)  # kInvalidArgument
    assert "hip" in msg and "cpu" in msg, msg


@pytest.mark.parametrize("op", ["add", "mul"])
def test_empty_graphs(dev, op):
    say(f"drop-in empty {op}")
    g = graphs.Graph("hip")
    x, y = g.input(F32, (0, 3)), g.input(F32, (0, 3))
    g.output(g.op(op, [x, y], (0, 3)))
    e = np.zeros((0, 3), np.float32)
    (got,), (want,) = both(g.text(), [e, e])
    assert got.shape == want.shape == (0, 3)


@pytest.mark.parametrize("dtype", [F32, F16, BF16])
@pytest.mark.parametrize("numel", [1023, 1024])
@pytest.mark.parametrize("op", ["add", "relu"])
def test_vectorization_boundary(dev, op, numel, dtype):
    say(f"drop-in {op} numel {numel} dtype {dtype}")
    g = graphs.Graph("hip")
    x = g.input(dtype, (numel,))
    if op == "add":
        y = g.input(dtype, (numel,))
        g.output(g.add(x, y))
        ins = [synth.tensor(61, (numel,), dtype, "normal"), synth.tensor(62, (numel,), dtype, "normal")]
    else:
        g.output(g.relu(x))
        ins = [synth.tensor(63, (numel,), dtype, "normal")]
    (got,), (want,) = both(g.text(), ins)
    assert_bitwise(got, want, f"{op} {numel} {dtype}")

"""ResNet-18 (C4) at its real shape, op by op, at the north star's per-op bf16 rule.

The whole-graph C4 tests compare end to end with a deep-graph criterion, because rounding differences of two
correct bf16 evaluations compound over 20 conv layers. This file closes that gap per op: C4's forward at batch 64,
224 px runs on hip as a chain of the subgraphs HipBackend::compile sees inside the full graph after the pass
pipeline (conv + bias with its relu epilogue; the second conv of a basic block with the residual add;relu
epilogue; the 1x1 stride-2 downsamples; both pools; the classifier GEMM with its bias add), each subgraph fed the
hip outputs of the ones before it. Every subgraph's output is then compared with the oracle's evaluation of the
same subgraph on identical inputs, images 0 and 63 of the batch (every op on the path computes each image
independently), at |a - e| <= 1e-2 * rms(e) + 1e-2 * |e| (tests/tolerance.py; reference rule
tests/cpp/common/tolerance.h:41-62,127). Reference semantics: src/backends/cpu/kernels/conv.cpp:223-314,
pool.cpp:210-350, matmul.cpp:92-185, fused_elementwise_utils.cpp:122-206.
"""
import numpy as np
import pytest

import oracle_lib as orc
from frame_hip import graphs, host
from tolerance import assert_close

pytestmark = pytest.mark.gpu
BF16 = 3
BATCH, IMAGE, CHECK = 64, 224, [0, 63]


def say(msg):
    print(f"[case] {msg}", flush=True)


def sub_conv(batch, device, xs, ws, stride, pad, relu=True, residual=False):
    """conv2d(x, w, b) [-> add(., identity)] [-> relu], the shape of one lowered conv node with its epilogue."""
    g = graphs.Graph(device)
    x = g.input(BF16, (batch,) + tuple(xs[1:]))
    w = g.input(BF16, ws)
    b = g.input(BF16, (ws[0],))
    y = g.conv2d(x, w, b, (stride, stride), (pad, pad))
    if residual:
        y = g.add(y, g.input(BF16, y.shape))
    if relu:
        y = g.relu(y)
    g.output(y)
    return g


def sub_pool(batch, device, xs, kind, k, s, p):
    g = graphs.Graph(device)
    x = g.input(BF16, (batch,) + tuple(xs[1:]))
    g.output(g.pool(kind, x, (k, k), (s, s), (p, p)))
    return g


def sub_fc(batch, device, features, classes):
    g = graphs.Graph(device)
    x = g.input(BF16, (batch, features))
    w = g.input(BF16, (features, classes))
    b = g.input(BF16, (batch, classes))
    g.output(g.add(g.matmul(x, w), b))
    return g


def c4_chain():
    """Runs C4 on hip as its chain of subgraphs. Yields (name, build(batch, device), inputs, hip output, per_row),
    per_row[i] telling whether input i has the batch as its first axis."""
    _, specs = graphs.resnet18(batch=BATCH, dtype=BF16, device="hip")
    ins = graphs.resnet18_inputs(specs, batch=BATCH, dtype=BF16)
    params = iter(ins[1:])

    def run(build, inputs):
        (out,) = host.compile(build(BATCH, "hip"), "hip").run(inputs)
        return out

    x = ins[0]
    w, b = next(params), next(params)
    build = lambda n, d, xs=x.shape, ws=w.shape: sub_conv(n, d, xs, ws, 2, 3)
    h = run(build, [x, w, b])
    yield "stem conv7x7/s2 + bias + relu", build, [x, w, b], h, [True, False, False]
    build = lambda n, d, xs=h.shape: sub_pool(n, d, xs, "max_pool2d", 3, 2, 1)
    x, h = h, run(build, [h])
    yield "max_pool2d 3x3/s2", build, [x], h, [True]
    for stage, cout in enumerate((64, 128, 256, 512)):
        for block in range(2):
            stride = 2 if (stage > 0 and block == 0) else 1
            tag = f"layer{stage + 1}.{block}"
            identity = h
            w1, b1, w2, b2 = next(params), next(params), next(params), next(params)
            build = lambda n, d, xs=h.shape, ws=w1.shape, s=stride: sub_conv(n, d, xs, ws, s, 1)
            y = run(build, [h, w1, b1])
            yield f"{tag} conv1 3x3/s{stride} + bias + relu", build, [h, w1, b1], y, [True, False, False]
            if stride != 1 or identity.shape[1] != cout:
                wd, bd = next(params), next(params)
                build = lambda n, d, xs=identity.shape, ws=wd.shape: sub_conv(n, d, xs, ws, 2, 0, relu=False)
                ds = run(build, [identity, wd, bd])
                yield f"{tag} downsample 1x1/s2 + bias", build, [identity, wd, bd], ds, [True, False, False]
                identity = ds
            build = lambda n, d, xs=y.shape, ws=w2.shape: sub_conv(n, d, xs, ws, 1, 1, residual=True)
            h = run(build, [y, w2, b2, identity])
            yield f"{tag} conv2 3x3 + bias, residual add;relu", build, [y, w2, b2, identity], h, [True, False, False, True]
    hw = h.shape[2]
    build = lambda n, d, xs=h.shape: sub_pool(n, d, xs, "avg_pool2d", hw, 1, 0)
    x, h = h, run(build, [h])
    yield f"avg_pool2d {hw}x{hw}", build, [x], h, [True]
    feats = h.reshape(BATCH, -1)
    wf, bf = next(params), next(params)
    build = lambda n, d: sub_fc(n, d, wf.shape[0], wf.shape[1])
    logits = run(build, [feats, wf, bf])
    yield "classifier matmul + bias", build, [feats, wf, bf], logits, [True, False, True]


def test_c4_resnet_every_op_at_1e2(request):
    assert host.device_count("hip") >= 1, "no hip device"
    orc.load_cpu_backend()
    counts = {"conv": 0, "residual": 0, "pool": 0, "fc": 0}
    for name, build, inputs, got, per_row in c4_chain():
        say(f"C4 op {name}: output {got.shape}")
        sub_ins = [a[CHECK] if r else a for a, r in zip(inputs, per_row)]
        (want,) = orc.run_graph_cpu(build(len(CHECK), "cpu"), sub_ins)
        stats = assert_close(got[CHECK], want, BF16, what=f"C4 {name}, images {CHECK}")
        say(f"  max |err| {stats['max_abs']:.3g} (atol {stats['atol']:.3g}) over {stats['n']} outputs")
        counts["conv"] += "conv" in name or "downsample" in name
        counts["residual"] += "residual" in name
        counts["pool"] += "pool" in name
        counts["fc"] += "classifier" in name
    assert counts == {"conv": 20, "residual": 8, "pool": 2, "fc": 1}, counts

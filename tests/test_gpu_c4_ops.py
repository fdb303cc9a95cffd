"""ResNet-18 (C4) at its real shape, op by op, at the north star's per-op bf16 rule.

The whole-graph C4 tests compare end to end with a deep-graph criterion, because rounding differences of two
correct bf16 evaluations compound over 20 conv layers. This file holds every op of C4's forward to the per-op rule
|a - e| <= 1e-2 * rms(e) + 1e-2 * |e| (tests/tolerance.py; reference rule tests/cpp/common/tolerance.h:41-62,127)
on images 0 and 63 of the batch (every op on the path computes each image independently), two ways:

* test_c4_full_graph_every_step_at_1e2: the real 224 px, batch-64 executable, i.e. the kernels C4 itself runs
  (the fused stem conv + relu + max pool, channels-last convs with out_nhwc epilogues, the band NCHW convs, the
  NHWC whole-plane average pool, the classifier GEMM with its bias epilogue). Every step's output is tapped as it is
  produced (frame_hip_run_tapped); each compute step is recomputed by the oracle from the tapped hip values of its
  operands (channels-last values converted on the host) and compared; the layout steps (C8 packs, filter and
  activation transposes) must equal their host counterparts bit for bit, and max pooling is a selection, so it
  is compared bit for bit as well.
* test_c4_resnet_every_op_at_1e2: the same network as a chain of separately compiled one-op subgraphs (conv + bias
  with its relu epilogue, the residual add;relu convs, the 1x1 downsamples, both pools, the classifier), each fed
  the hip outputs of the ones before it. These subgraphs lower to NCHW-output kernels with channels-last copies
  of their inputs, not to the instances the full graph runs; they check the op semantics at full size.

Reference semantics: src/backends/cpu/kernels/conv.cpp:223-314, pool.cpp:210-350, matmul.cpp:92-185,
fused_elementwise_utils.cpp:122-206.
"""
import re

import numpy as np
import pytest

import oracle_lib as orc
from frame_hip import graphs, host
from tolerance import assert_bitwise, assert_close

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


# ---- the full graph, every step tapped ------------------------------------------------------------------------

NODE = re.compile(r"^(?P<outs>%[\d, %]+) = (?P<op>\w+)\((?P<ins>[^)]*)\)(?: \{(?P<attrs>.*)\})? : (?P<types>.*)$")
TYPE = re.compile(r"(\w+)\[([\d,]*)\]@")
ATTR = re.compile(r"(\w+)=(\[[^\]]*\]|[^,}]+)")
EW_ADD, EW_RELU = 1, 3


def parse_lowered(text):
    """Non-input nodes of the lowered graph text: (output ids, op, input ids, attrs, [(dtype name, shape)])."""
    nodes = []
    for line in text.splitlines():
        m = NODE.match(line)
        if m is None or m["op"] == "graph_input":
            continue
        outs = [int(t) for t in re.findall(r"%(\d+)", m["outs"])]
        ins = [int(t) for t in re.findall(r"%(\d+)", m["ins"])]
        attrs = {}
        for k, v in ATTR.findall(m["attrs"] or ""):
            v = v.strip()
            attrs[k] = [int(x) for x in v[1:-1].split(",") if x.strip()] if v.startswith("[") else int(v)
        types = [(dt, tuple(int(d) for d in dims.split(",") if d)) for dt, dims in TYPE.findall(m["types"])]
        assert len(types) == len(outs), line
        nodes.append((outs, m["op"], ins, attrs, types))
    return nodes


def test_c4_full_graph_every_step_at_1e2():
    assert host.device_count("hip") >= 1, "no hip device"
    g, specs = graphs.resnet18(batch=BATCH, dtype=BF16, device="hip")
    ins = graphs.resnet18_inputs(specs, batch=BATCH, dtype=BF16)
    text = g.text()
    exe = host.compile(text, "hip", 1)
    nodes = parse_lowered(host.hip_lowered(text, 1))
    assert exe.steps() == [op for _, op, _, _, _ in nodes], "plan steps differ from the lowered graph's nodes"
    say(f"C4 full graph: {len(nodes)} steps")

    # every output of every step, tapped (the float32 ones are split-K workspaces of layer-4 convs)
    values, taps = {}, []
    for step, (outs, op, _, _, types) in enumerate(nodes):
        for j, (oid, (dt, shape)) in enumerate(zip(outs, types)):
            values[oid] = np.empty(shape, np.float32 if dt in ("f32", "float32") else np.uint16)
            taps.append((step, j, values[oid]))
    n_in = len(ins)
    for i, a in enumerate(ins):
        values[i] = a
    t_in = exe.upload_inputs(ins)
    t_out = exe.alloc_outputs()
    stream = host.Stream("hip")
    exe.run_tapped(t_in, t_out, stream, taps)
    (logits,) = [o.numpy() for o in t_out]
    assert_bitwise(logits, values[nodes[-1][0][0]], "graph output vs the last step's tap")

    # layout of every value: graph inputs NCHW; "nhwc" values [N,H,W,C]; C8 packs; [N,C] after the folded pool
    layout = {i: "nchw" for i in range(n_in)}
    source = {}  # a transposed / packed filter -> the graph-input filter it came from

    def nchw(vid):
        a, lay = values[vid], layout[vid]
        return a if lay == "nchw" else np.ascontiguousarray(np.transpose(a, (0, 3, 1, 2)))

    counts = {}
    for outs, op, args, attrs, types in nodes:
        counts[op] = counts.get(op, 0) + 1
        out = outs[0]
        if op == "hip_pack_input_c8_internal":
            x = values[args[0]]
            want = np.zeros(x.shape[:1] + x.shape[2:] + (8,), np.uint16)
            want[..., :x.shape[1]] = np.transpose(x, (0, 2, 3, 1))
            assert_bitwise(values[out][CHECK], want[CHECK], "C8 input pack")
            layout[out], source[out] = "c8", args[0]
        elif op == "hip_pack_filter_c8_internal":
            w = values[args[0]]
            co, c, kh, kw = w.shape
            want = np.zeros(types[0][1], np.uint16)
            want[:, :kh * kw * 8].reshape(co, kh * kw, 8)[:, :, :c] = np.transpose(w.reshape(co, c, kh * kw), (0, 2, 1))
            assert_bitwise(values[out], want, "C8 filter pack")
            layout[out], source[out] = "c8", args[0]
        elif op in ("hip_channels_last_multi_internal", "hip_channels_last_internal"):
            for a, o in zip(args, outs):
                x = values[a]
                rows = CHECK if a not in range(1, n_in) else slice(None)
                assert_bitwise(values[o][rows], np.transpose(x, (0, 2, 3, 1))[rows], f"{op} of %{a}")
                layout[o] = "nhwc"
                source[o] = source.get(a, a)
        elif op == "hip_conv2d_nhwc_internal":
            xid, wid, bid = args[0], args[1], args[2]
            x = values[source[xid]][CHECK] if layout[xid] == "c8" else nchw(xid)[CHECK]
            w = values[source.get(wid, wid)]
            assert w.ndim == 4 and source.get(wid, wid) < n_in, "filter traced to a graph input"
            kh, kw = attrs["filter_hw"]
            (sh, sw), (ph, pw) = attrs["stride"], attrs["padding"]
            geom = (len(CHECK), x.shape[1], x.shape[2], x.shape[3], w.shape[0], kh, kw, sh, sw, ph, pw, 1)
            want = orc.conv2d(BF16, np.ascontiguousarray(x), w, values[bid], geom)
            prog = attrs.get("ep_ops", [])
            if prog:
                operands = [want] + [nchw(r)[CHECK] for r in args[3:]]
                want = orc.ew_program(BF16, prog, [2 if p == EW_ADD else 1 for p in prog], operands)
            layout[out] = "nhwc" if attrs.get("out_nhwc", 0) else "nchw"
            tag = (f"conv {kh}x{kw}/s{sh} {x.shape[1]}->{w.shape[0]} at {x.shape[2]}x{x.shape[3]} "
                   f"{'c8 ' if layout[xid] == 'c8' else ''}{'in_nchw ' if attrs.get('in_nchw') else ''}"
                   f"{'w_oihw ' if attrs.get('w_oihw') else ''}{layout[out]} out, epilogue {prog}")
            st = assert_close(nchw(out)[CHECK], want, BF16, what=f"C4 step %{out}: {tag}")
            say(f"  %{out} {tag}: max |err| {st['max_abs']:.3g} (atol {st['atol']:.3g})")
        elif op == "hip_conv2d_stem_pool_internal":
            # the stem conv 7x7/2 + bias, relu and the 3x3/2 max pool in one kernel; the conv output is never stored
            x, w, b = values[args[0]][CHECK], values[args[1]], values[args[2]]
            (sh, sw), (ph, pw) = attrs["stride"], attrs["padding"]
            geom = (len(CHECK), x.shape[1], x.shape[2], x.shape[3], w.shape[0], 7, 7, sh, sw, ph, pw, 1)
            conv = orc.conv2d(BF16, np.ascontiguousarray(x), w, b, geom)
            if attrs["relu"]:
                conv = orc.ew_program(BF16, [EW_RELU], [1], [conv])
            (kh, kw), (psh, psw), (pph, ppw) = attrs["kernel"], attrs["pool_stride"], attrs["pool_padding"]
            want = orc.pool2d(BF16, 0, conv, conv.shape + (kh, kw, psh, psw, pph, ppw))
            layout[out] = "nchw"
            st = assert_close(values[out][CHECK], want, BF16, what=f"C4 step %{out}: stem conv + relu + max pool")
            say(f"  %{out} stem conv 7x7/2 + relu + max pool 3x3/2: max |err| {st['max_abs']:.3g}")
        elif op in ("max_pool2d", "hip_max_pool2d_nhwc_internal"):
            x = nchw(args[0])[CHECK]
            (kh, kw), (sh, sw), (ph, pw) = attrs["kernel"], attrs["stride"], attrs["padding"]
            want = orc.pool2d(BF16, 0, np.ascontiguousarray(x), (len(CHECK),) + x.shape[1:] + (kh, kw, sh, sw, ph, pw))
            layout[out] = "nchw" if op == "max_pool2d" else "nhwc"
            assert_bitwise(nchw(out)[CHECK], want, f"C4 step %{out}: {op}")
            say(f"  %{out} {op}: bit-exact")
        elif op == "hip_avg_pool2d_nhwc_internal":
            x = nchw(args[0])[CHECK]
            (kh, kw), (sh, sw), (ph, pw) = attrs["kernel"], attrs["stride"], attrs["padding"]
            want = orc.pool2d(BF16, 1, np.ascontiguousarray(x), (len(CHECK),) + x.shape[1:] + (kh, kw, sh, sw, ph, pw))
            layout[out] = "flat"
            assert_bitwise(values[out][CHECK], want.reshape(len(CHECK), -1), f"C4 step %{out}: global average pool")
            say(f"  %{out} {op}: bit-exact")
        elif op == "hip_matmul_epilogue_internal":
            a, w, b = values[args[0]][CHECK], values[args[1]], values[args[2]][CHECK]
            prog = attrs.get("ep_ops", [])
            assert prog == [EW_ADD], prog
            want = orc.ew_program(BF16, [EW_ADD], [2], [orc.matmul(BF16, np.ascontiguousarray(a), w), b])
            layout[out] = "flat"
            st = assert_close(values[out][CHECK], want, BF16, what=f"C4 step %{out}: classifier")
            say(f"  %{out} classifier matmul + bias: max |err| {st['max_abs']:.3g}")
        else:
            raise AssertionError(f"step {op} has no check")
    say(f"C4 full graph steps checked: {counts}")
    stem = counts.get("hip_conv2d_stem_pool_internal", 0)
    assert counts.get("hip_conv2d_nhwc_internal", 0) + stem == 20, counts
    assert counts.get("hip_avg_pool2d_nhwc_internal", 0) == 1 and counts.get("hip_matmul_epilogue_internal", 0) == 1
    assert counts.get("max_pool2d", 0) + counts.get("hip_max_pool2d_nhwc_internal", 0) + stem == 1

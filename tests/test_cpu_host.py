"""The C++20 host side (libframe.so) on the CPU: the C ABI surface, the nine-pass pipeline against the
reference's own golden IR fixtures (tests/golden/compiler, copied from the reference's
tests/cpp/compiler/testdata) and against the reference pipeline itself, the memory plan, the compile cache and
the error contract. No GPU is touched: graphs here live on the oracle's `cpu` backend, and hip graphs stop
before Backend::compile."""
import ctypes
import os
import re
import subprocess

import pytest

import oracle_lib as orc
from frame_hip import abi, graphs, host

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(REPO, "tests", "golden", "compiler")
needs_ref = pytest.mark.skipif(not orc.ref_available(), reason="oracle/_ref not built (no /root/reference here)")

PASS_OF_PREFIX = {
    "add_passthrough": "backend_lowering",
    "canonicalize": "canonicalize",
    "constant_folding": "constant_folding",
    "cse": "common_subexpression_elimination",
    "dne": "dead_node_elimination",
    "layout_assignment": "layout_assignment",
    "memory_planning": "memory_planning",
    "operator_fusion": "operator_fusion",
}


def golden_cases():
    cases = []
    for f in sorted(os.listdir(GOLDEN)):
        if not f.endswith("_input.txt"):
            continue
        stem = f[: -len("_input.txt")]
        expected = os.path.join(GOLDEN, stem + "_expected.txt")
        if not os.path.exists(expected):
            continue
        prefix = next(p for p in PASS_OF_PREFIX if stem.startswith(p))
        cases.append((stem, PASS_OF_PREFIX[prefix]))
    return cases


def read(name):
    with open(os.path.join(GOLDEN, name)) as fh:
        return fh.read()


def declared(header, pattern):
    with open(os.path.join(REPO, "include", header)) as fh:
        text = fh.read()
    return sorted(set(re.findall(pattern, text)))


def exported(lib_path):
    out = subprocess.run(["nm", "-D", "--defined-only", lib_path], check=True, capture_output=True, text=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_kernel_abi_library_exports_every_declared_symbol():
    syms = declared("frame_hip_abi.h", r"\b(fh_[a-z0-9_]+)\s*\(")
    assert len(syms) >= 25
    have = exported(abi.KERNELS_LIB)
    assert not [s for s in syms if s not in have], "missing kernel ABI symbols"
    abi.lib()  # loads (no device call)
    assert set(abi.exported_symbols()) <= set(syms)


def test_host_library_exports_every_declared_symbol():
    syms = declared("frame_capi.h", r"\b(frame_[a-z0-9_]+)\s*\(")
    assert len(syms) >= 25
    have = exported(host.HOST_LIB)
    assert not [s for s in syms if s not in have], "missing host C API symbols"
    host.lib()
    assert set(host.exported_symbols()) == set(syms)


def test_hip_backend_is_registered_through_the_hal():
    assert "hip" in host.backends()


@pytest.fixture(scope="module")
def cpu_backend():
    orc.load_cpu_backend()


@pytest.mark.parametrize("stem,pass_name", golden_cases())
def test_pass_matches_reference_golden(cpu_backend, stem, pass_name):
    if stem.startswith("dne_side_effect"):
        pytest.skip("needs the reference's test-only op test_side_effect_op")
    got = host.transform(read(stem + "_input.txt"), pass_name)
    assert got == read(stem + "_expected.txt")


@pytest.mark.parametrize("stem", [s for s, _ in golden_cases()])
def test_text_round_trip(stem):
    text = read(stem + "_input.txt")
    if "test_side_effect_op" in text:
        pytest.skip("test-only op")
    assert host.roundtrip(text) == text


def sample_graph_texts():
    g1 = graphs.mlp(batch=8, dtype=0, device="cpu").text()
    g2, _ = graphs.resnet18(batch=1, dtype=3, device="cpu", image=32, classes=10)
    g3, _ = graphs.transformer_block(batch=2, seq=16, d_model=32, heads=2, ffn=64, dtype=3, device="cpu")
    g4 = graphs.conv(0, device="cpu", n=1, cin=4, h=6, w=6, cout=4).text()
    return {"mlp": g1, "resnet": g2.text(), "transformer_relu": g3.text().replace(" gelu(", " relu("), "conv": g4}


@needs_ref
@pytest.mark.parametrize("name", ["mlp", "resnet", "transformer_relu", "conv"])
def test_standard_pipeline_matches_reference(cpu_backend, name):
    text = sample_graph_texts()[name]
    assert host.transform(text) == orc.ref_transform(text)


@needs_ref
@pytest.mark.parametrize("name", ["mlp", "resnet", "transformer_relu", "conv"])
def test_memory_plan_matches_reference(cpu_backend, name):
    text = host.transform(sample_graph_texts()[name])
    assert host.memory_plan(text) == orc.ref_memory_plan(text)


def test_gelu_chain_fuses_on_hip():
    # add(matmul, bias) -> gelu becomes one fused group for the hip backend
    g, _ = graphs.transformer_block(batch=1, seq=8, d_model=16, heads=2, ffn=32, dtype=3, device="hip")
    out = host.transform(g.text())
    assert 'ops="add;gelu"' in out and 'ops="add;add"' in out
    assert out.count("constant(") == 1  # CSE merged the per-head scale constants


def test_compile_cache_hits(cpu_backend):
    text = graphs.mlp(batch=4, dtype=0, device="cpu").text()
    host.compile(text, "cpu")
    n = host.compile_cache_size()
    host.compile(text, "cpu")
    assert host.compile_cache_size() == n
    host.compile(text, "cpu", opt_level=0)  # options are part of the key
    assert host.compile_cache_size() == n + 1


def test_unknown_backend_is_not_found():
    with pytest.raises(host.FrameError) as e:
        host.compile(graphs.mlp(batch=2, device="cpu").text(), "no_such_backend")
    assert e.value.code == host.CODES["invalid_argument"]  # device/backend mismatch is checked first
    g = graphs.Graph("cpu")
    x = g.input(0, (2,))
    g.output(g.relu(x))
    with pytest.raises(host.FrameError) as e:
        host.transform(g.text().replace("@cpu:0", "@ascend:0"))
    assert e.value.code == host.CODES["not_found"]


def test_every_op_has_a_hip_kernel():
    """backend_lowering (the last pass) finds a `hip` kernel for every op this build registers, the training
    path's gradient ops and the unary ops their micrographs use included (a missing one is kUnimplemented, named)."""
    g = graphs.Graph("hip")
    x = g.input(0, (4, 8))
    y = g.input(0, (4, 8))
    outs = [g.op(op, [x], (4, 8)) for op in ("sigmoid", "tanh", "rsqrt", "gelu", "relu", "square")]
    outs += [g.op(op, [x, y], (4, 8)) for op in ("relu_grad_internal", "gelu_grad_internal", "add", "mul")]
    for o in outs:
        g.output(o)
    host.transform(g.text())  # standard pipeline for "hip": raises FrameError(unimplemented) on a missing kernel


def test_shape_inference_rejects_inconsistent_types():
    g = graphs.Graph("cpu")
    a = g.input(0, (2, 3))
    b = g.input(0, (4, 5))
    g.output(g.op("matmul", [a, b], (2, 5)))
    with pytest.raises(host.FrameError) as e:
        host.transform(g.text())
    assert "contraction dimension mismatch" in str(e.value)


# ---- attention lowering (host only: the graph HipBackend::compile plans) ----------------------------------

def attention_graph(batch=2, seq=64, heads=2, dh=64, dtype=3, swap_mul=False, head_order=None, leak=False,
                    scale=None):
    """Q, K, V inputs -> the reference's per-(batch, head) decomposition (src/nn/layers.cpp:1014-1080)."""
    g = graphs.Graph("hip")
    rows, width = batch * seq, heads * dh
    q, k, v = (g.input(dtype, (rows, width)) for _ in range(3))
    c = g.constant_splat(dtype, (seq, seq), (1.0 / dh ** 0.5) if scale is None else scale)
    per_batch = []
    for b in range(batch):
        qr, kr, vr = (g.slice(t, 0, b * seq, (b + 1) * seq) for t in (q, k, v))
        outs = []
        for h in (head_order or range(heads)):
            qh, kh, vh = (g.slice(t, 1, h * dh, (h + 1) * dh) for t in (qr, kr, vr))
            s = g.matmul(qh, g.transpose(kh, (1, 0)))
            s = g.mul(c, s) if swap_mul else g.mul(s, c)
            p = g.softmax(s)
            if leak and b == 0 and h == 0:
                g.output(p)
            outs.append(g.matmul(p, vh))
        per_batch.append(g.concat(outs, 1))
    g.output(g.concat(per_batch, 0))
    return g


def test_attention_decomposition_lowers_to_one_node():
    for opt in (0, 1, 2):
        out = host.hip_lowered(attention_graph().text(), opt)
        ops = re.findall(r"= (\w+)\(", out)
        assert ops == ["graph_input"] * 3 + ["hip_attention_internal"], out
        assert "batch=2" in out and "seq=64" in out and "heads=2" in out and "dh=64" in out and "scale=0.125" in out


def test_attention_lowering_accepts_either_mul_operand_order():
    assert "hip_attention_internal" in host.hip_lowered(attention_graph(swap_mul=True).text())


def test_attention_scale_is_the_constant_narrowed_to_the_dtype():
    # 0.1 is not a bfloat16; the kernel must see the value the constant node stores (0.10009765625)
    out = host.hip_lowered(attention_graph(scale=0.1).text())
    assert "scale=0.10009765625" in out, out


@pytest.mark.parametrize("kwargs", [
    {"leak": True},                 # a probability matrix is also a graph output
    {"head_order": [1, 0]},         # heads concatenated out of order
    {"dh": 32, "heads": 4},         # head dim the kernel does not take
    {"seq": 48},                    # sequence not a multiple of 64
    {"seq": 576, "batch": 1},       # sequence beyond 512
    {"dtype": 0},                   # float32 keeps the decomposition
])
def test_attention_lowering_keeps_the_decomposition_when_it_cannot_apply(kwargs):
    out = host.hip_lowered(attention_graph(**kwargs).text())
    assert "hip_attention_internal" not in out and "softmax" in out


def test_attention_support_query_is_host_only():
    lib = abi.lib()
    assert lib.fh_attention_supported(3, 512, 64) == 1 and lib.fh_attention_supported(2, 64, 64) == 1
    assert lib.fh_attention_supported(0, 512, 64) == 0 and lib.fh_attention_supported(3, 512, 128) == 0
    assert lib.fh_attention_supported(3, 100, 64) == 0 and lib.fh_attention_supported(3, 1024, 64) == 0


def test_wgrad_workspace_rejects_invalid_geometry_on_the_host():
    """fh_conv2d_wgrad_workspace validates before it divides: zero strides, negative padding, zero extents and a
    filter larger than the padded input give -1 (no SIGFPE, no truncated output size); host-only."""
    lib = abi.lib()

    def ws(geom):
        return lib.fh_conv2d_wgrad_workspace(3, abi.i64_array(geom), 64, None)

    good = [32, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1]
    assert ws(good) > 0
    for k, v in [(7, 0), (8, 0), (7, -1), (9, -1), (10, -2), (0, 0), (2, 0), (5, 0)]:
        bad = list(good)
        bad[k] = v
        assert ws(bad) == -1, (k, v)
    assert ws([1, 64, 2, 2, 64, 5, 5, 1, 1, 1, 1, 1]) == -1  # h + 2p < kh
    assert ws([1, 64, 8, 2, 64, 3, 5, 1, 1, 1, 1, 1]) == -1  # w + 2p < kw


def test_conv_split_k_plan_is_host_only():
    """fh_conv2d_nhwc_split_workspace plans split K on the host: ResNet-18's 7x7x512 3x3 convs at batch 64 split in
    two (100 tiles of 128 x 128 for 256 CUs, 144 k stages), the stride-2 one (72 stages), layer 3 (Cout 256) and
    fp32 stay unsplit; an explicit count is reduced so no split is empty; NCHW output and Cout % 128 give -1."""
    lib = abi.lib()
    k = ctypes.c_int32(0)

    def plan(geom, dtype=3, flags=1, splits=0):
        k.value = splits
        return lib.fh_conv2d_nhwc_split_workspace(dtype, abi.i64_array(geom), flags, ctypes.byref(k)), k.value

    l4 = (64, 512, 7, 7, 512, 3, 3, 1, 1, 1, 1, 1)
    assert plan(l4) == (2 * 3136 * 512 * 4, 2)
    assert plan((64, 256, 14, 14, 512, 3, 3, 2, 2, 1, 1, 1)) == (0, 0)  # stride 2: K = 2304
    assert plan((64, 256, 14, 14, 256, 3, 3, 1, 1, 1, 1, 1)) == (0, 0)
    assert plan((256, 512, 7, 7, 512, 3, 3, 1, 1, 1, 1, 1)) == (0, 0)  # 392 tiles: no split fits one round
    assert plan(l4, dtype=0) == (0, 0)
    assert plan(l4, splits=5) == (5 * 3136 * 512 * 4, 5)
    assert plan(l4, splits=100) == (72 * 3136 * 512 * 4, 72)  # 144 stages: 2 per split
    assert plan(l4, flags=0, splits=2)[0] == -1 and plan(l4, dtype=0, splits=2)[0] == -1
    assert plan((64, 512, 7, 7, 320, 3, 3, 1, 1, 1, 1, 1), splits=2)[0] == -1
    assert lib.fh_conv2d_nhwc_split_workspace(3, None, 1, ctypes.byref(k)) == -1


def test_resnet_layer4_lowers_with_split_k_workspaces():
    # at batch 64 the three 3x3 stride-1 convs of layer 4 carry their fp32 partials as a second planned output
    g, _ = graphs.resnet18(batch=64, dtype=3)
    out = host.hip_lowered(g.text(), 1)
    ws = [l for l in out.splitlines() if "hip_conv2d_nhwc_internal" in l and "float32[3211264]" in l]
    assert len(ws) == 3, ws
    assert all("out_nhwc=1" in l and "[64,7,7,512]" in l for l in ws)


@pytest.mark.parametrize("dtype,cin,lowered", [(3, 64, "hip_conv2d_nhwc_internal"), (0, 64, "hip_conv2d_nhwc_internal"),
                                               (3, 3, "hip_pack_input_c8_internal"), (0, 3, "conv2d"),
                                               (0, 24, "conv2d")])
def test_conv_lowering_by_dtype_and_channels(dtype, cin, lowered):
    # bf16 and fp32 with a stage-aligned channel count go channels-last; a bf16 stem takes the C8 packing;
    # fp32 with 3 or 24 channels keeps the direct conv
    g = graphs.conv(dtype, device="hip", n=1, cin=cin, h=12, w=12, cout=32, k=3)
    out = host.hip_lowered(g.text(), 1)
    assert lowered in out, out
    if lowered == "conv2d":
        assert "hip_conv2d_nhwc_internal" not in out


def test_resnet_lowering_layouts():
    # every conv filter that needs it is transposed in one batched channels-last step; the 56x56 (here 16x16) layer's
    # four convs are band convs (Cin 64, Cout 64, 3x3): that layer, the stem's output and the max pool stay NCHW and
    # those convs read their filters as they are (w_oihw); everything after it is channels-last, with one
    # channels-last copy of the layer's output for the next layer's two convs
    g, _ = graphs.resnet18(batch=2, dtype=3, image=64)
    out = host.hip_lowered(g.text(), 1)
    ops = re.findall(r"= (\w+)\(", out)
    assert ops.count("hip_channels_last_multi_internal") == 1
    assert ops.count("hip_conv2d_nhwc_internal") == 19  # the stem conv is fused with its relu and max pool
    assert ops.count("hip_conv2d_stem_pool_internal") == 1 and "relu=1" in out
    assert out.count("w_oihw=1") == 4 and out.count("in_nchw=1") == 4
    assert ops.count("hip_channels_last_internal") == 1
    assert ops.count("max_pool2d") == 0 and ops.count("hip_avg_pool2d_nhwc_internal") == 1
    assert ops.count("reshape") == 0  # the global pool writes [N, C] itself
    assert ops.count("graph_input") == 43
    assert out.count("out_nhwc=1") == 15


@pytest.mark.parametrize("opt_level", [0, 1])
def test_stem_pool_lowering(opt_level):
    # conv2d 7x7/2 -> relu -> max_pool2d 3x3/2 becomes one fused node at every opt level (bf16, Cin 3, Cout 64);
    # fp32 keeps the three nodes, and so does a graph that also outputs the conv result
    def stem(dtype, also_output=False):
        g = graphs.Graph("hip")
        x = g.input(dtype, (2, 3, 64, 64))
        w, b = g.input(dtype, (64, 3, 7, 7)), g.input(dtype, (64,))
        c = g.conv2d(x, w, b, (2, 2), (3, 3))
        r = g.relu(c)
        g.output(g.pool("max_pool2d", r, (3, 3), (2, 2), (1, 1)))
        if also_output:
            g.output(c)
        return host.hip_lowered(g.text(), opt_level)
    out = stem(3)
    assert "hip_conv2d_stem_pool_internal" in out and "relu=1" in out and "max_pool2d(" not in out, out
    assert "hip_conv2d_stem_pool_internal" not in stem(0)
    assert "hip_conv2d_stem_pool_internal" not in stem(3, also_output=True)


def test_training_lowering_keeps_band_layer_channels_last():
    # the NCHW preference for band convs applies to forward graphs only: a training graph's layout plan is unchanged
    g, specs = graphs.resnet18(batch=2, dtype=3, image=64, train=True)
    text = host.backward(g.text(), 0, list(range(1, len(specs) + 1)))
    out = host.hip_lowered(text, 1)
    assert "w_oihw=1" not in out


def _conv_chain(last_is_output=True, softmax_tail=False):
    g = graphs.Graph("hip")
    x = g.input(3, (2, 32, 10, 10))
    w1, w2 = g.input(3, (32, 32, 3, 3)), g.input(3, (32, 32, 3, 3))
    a = g.relu(g.conv2d(x, w1, padding=(1, 1)))
    b = g.conv2d(a, w2, padding=(1, 1))
    if softmax_tail:
        g.output(g.softmax(g.reshape(b, (2 * 32 * 10, 10))))
    else:
        g.output(b)
    return g


def test_channels_last_stops_at_graph_outputs_and_other_uses():
    # the first conv's result feeds the second conv only: channels-last; the second is a graph output: NCHW
    out = host.hip_lowered(_conv_chain().text(), 1)
    assert out.count("out_nhwc=1") == 1 and "hip_channels_last_internal" in out  # x of the first conv
    # a reshape of a non-1x1 plane needs NCHW order: the second conv stays NCHW
    out = host.hip_lowered(_conv_chain(softmax_tail=True).text(), 1)
    assert out.count("out_nhwc=1") == 1


def test_qkv_projections_become_one_grouped_gemm():
    # the three projections of the attention block read the LN1 output: one grouped node at opt_level 1, with the
    # bias adds as per-group epilogues; opt_level 0 keeps three matmuls; fp32 is left alone
    g, _ = graphs.transformer_block(batch=2, seq=128, d_model=128, heads=2, ffn=256, dtype=3)
    out = host.hip_lowered(g.text(), 1)
    ops = re.findall(r"= (\w+)\(", out)
    assert ops.count("hip_matmul_grouped_internal") == 1, out
    line = [l for l in out.splitlines() if "hip_matmul_grouped_internal" in l][0]
    assert "groups=3" in line and "ep_ops=[1]" in line and "any_order=1" in line
    assert line.count("bfloat16[256,128]") == 3  # three outputs
    assert ops.count("hip_matmul_epilogue_internal") == 3  # output projection, FFN up, FFN down
    assert "hip_matmul_grouped_internal" not in host.hip_lowered(g.text(), 0)
    g32, _ = graphs.transformer_block(batch=1, seq=64, d_model=128, heads=2, ffn=256, dtype=0)
    assert "hip_matmul_grouped_internal" not in host.hip_lowered(g32.text(), 1)


def test_grouping_skips_members_that_depend_on_each_other():
    # y2's bias is y1 itself: merging would make the group read its own output, so the two stay apart
    g = graphs.Graph("hip")
    x, w1, w2, b1 = g.input(3, (64, 64)), g.input(3, (64, 64)), g.input(3, (64, 64)), g.input(3, (64, 64))
    y1 = g.add(g.matmul(x, w1), b1)
    y2 = g.add(g.matmul(x, w2), y1)
    g.output(y2)
    out = host.hip_lowered(g.text(), 1)
    assert "hip_matmul_grouped_internal" not in out
    # independent members with equal shapes and programs do merge, up to four per node
    g = graphs.Graph("hip")
    x = g.input(3, (64, 64))
    ws = [g.input(3, (64, 32)) for _ in range(5)]  # operands must precede the first member in topological order
    ys = [g.relu(g.matmul(x, w)) for w in ws]
    for y in ys:
        g.output(y)
    out = host.hip_lowered(g.text(), 1)
    ops = re.findall(r"= (\w+)\(", out)
    assert ops.count("hip_matmul_grouped_internal") == 1 and "groups=4" in out
    assert ops.count("hip_matmul_epilogue_internal") == 1  # the fifth


def test_small_fused_gemms_are_marked_any_order_only_above_opt0():
    # C1 at opt_level 1: two fused GEMMs that may reassociate k, the classifier's softmax folded into the second
    g = graphs.mlp(64, 0)
    out = host.hip_lowered(g.text(), 1)
    assert out.count("any_order=1") == 2 and out.count("row_softmax=1") == 1 and "softmax(" not in out, out
    out0 = host.hip_lowered(g.text(), 0)
    assert "any_order" not in out0 and "row_softmax" not in out0 and "softmax(" in out0


def test_softmax_fold_needs_a_narrow_single_use_gemm():
    def build(n, extra_use):
        g = graphs.Graph("hip")
        x, w, b = g.input(0, (8, 32)), g.input(0, (32, n)), g.input(0, (8, n))
        y = g.add(g.matmul(x, w), b)
        g.output(g.softmax(y))
        if extra_use:
            g.output(y)
        return host.hip_lowered(g.text(), 1)
    assert "row_softmax=1" in build(16, False)
    assert "row_softmax" not in build(17, False)  # wider than one split-k tile
    assert "row_softmax" not in build(10, True)   # the GEMM result is also a graph output


def test_gemm_grouped_and_ex_argument_checks():
    # validation happens before any device call, so it runs without a GPU
    lib = abi.lib()
    ptrs = (ctypes.c_void_p * 4)(8, 8, 8, 8)
    eps = (abi.Epilogue * 4)()
    for groups in (0, 5):
        assert lib.fh_gemm_grouped(3, 8, groups, ptrs, ptrs, 64, 64, 64, eps, 1, None) == 1  # invalid_argument
    eps[0] = abi.make_epilogue([(abi.EW_ADD, 8)])
    eps[1] = abi.make_epilogue([(abi.EW_MUL, 8)])
    assert lib.fh_gemm_grouped(3, 8, 2, ptrs, ptrs, 64, 64, 64, eps, 1, None) == 1
    assert b"different epilogue programs" in lib.fh_last_error()
    assert lib.fh_gemm_grouped(3, 8, 2, ptrs, ptrs, 64, 64, 64, eps, 4, None) == 1  # unknown flag
    assert lib.fh_gemm_ex(3, 8, 8, 8, 64, 64, 64, None, 6, None) == 1
    assert b"unknown flags" in lib.fh_last_error()


def test_nchw_graph_input_conv_reads_nchw_directly():
    # C3: the 3x3 stride-1 conv of a graph-input activation reads it NCHW (no channels-last copy of x, only of the
    # filter); a width the 8-pixel groups do not divide keeps the copy
    # and its filter in the graph's [Cout,Cin,KH,KW] layout too (the band kernel: no channels-last copy at all)
    out = host.hip_lowered(graphs.conv(3).text(), 1)
    assert out.count("hip_channels_last_internal(") == 0 and "in_nchw=1" in out and "w_oihw=1" in out, out
    out = host.hip_lowered(graphs.conv(3, w=57).text(), 1)
    assert out.count("hip_channels_last_internal(") == 2 and "in_nchw" not in out and "w_oihw" not in out, out
    lib = abi.lib()
    assert lib.fh_conv2d_nchw_in_supported(3, abi.i64_array([32, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1])) == 1
    assert lib.fh_conv2d_nchw_in_supported(3, abi.i64_array([32, 64, 56, 57, 64, 3, 3, 1, 1, 1, 1, 1])) == 0
    assert lib.fh_conv2d_nchw_in_supported(0, abi.i64_array([32, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1])) == 0
    c3 = abi.i64_array([32, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1])
    relu = abi.make_epilogue([(abi.EW_RELU, None)])
    gelu = abi.make_epilogue([(abi.EW_GELU, None)])
    assert lib.fh_conv2d_w_oihw_supported(3, c3, None) == 1
    assert lib.fh_conv2d_w_oihw_supported(3, c3, ctypes.byref(relu)) == 1
    assert lib.fh_conv2d_w_oihw_supported(3, c3, ctypes.byref(gelu)) == 0     # a program without a band instance
    assert lib.fh_conv2d_w_oihw_supported(2, c3, None) == 0                   # f16
    for g in ([32, 96, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1],                        # Cin 96
              [32, 64, 56, 56, 128, 3, 3, 1, 1, 1, 1, 1],                       # Cout 128
              [32, 64, 56, 57, 64, 3, 3, 1, 1, 1, 1, 1]):                       # W % 8 != 0
        assert lib.fh_conv2d_w_oihw_supported(3, abi.i64_array(g), None) == 0, g

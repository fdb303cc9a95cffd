"""The `hip` backend's HAL contract and runtime behaviour on the MI355X: Backend::copy round trips, kUnimplemented
for an op without a kernel, the eager hop (every node through Backend::launch, as the reference's
FallbackExecutable runs a graph) against the oracle, eager conv2d on MFMA, and the lifetime rules of the caching
allocator and the per-stream arenas (bounded memory over many run_with_allocated_outputs calls, no reuse of a
block that queued work still writes).

Reference contracts: tests/cpp/hal_conformance/test_hal_conformance.cpp:190-269 (copies, unsupported op),
src/runtime/fallback_executable.cpp:74-126,465 (node-by-node launch), src/runtime/compile.cpp:180-220
(run_with_allocated_outputs), src/backends/cuda/cuda_allocator.cpp:26-66 (free synchronises).
"""
import ctypes
import re

import numpy as np
import pytest

import oracle_lib as orc
from frame_hip import abi, graphs, host, synth
from tolerance import assert_bitwise, assert_close

pytestmark = pytest.mark.gpu
F32, F16, BF16 = 0, 2, 3


def say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def dev():
    assert host.device_count("hip") >= 1, "no hip device"
    orc.load_cpu_backend()


# ---- HAL conformance --------------------------------------------------------------------------------------

def test_copy_round_trips_h2d_d2d_d2h_h2h(dev):
    say("Backend::copy H2D -> D2D -> D2D -> D2H, then H2H, with and without a stream")
    n = 128
    pattern = (np.arange(n, dtype=np.uint32) * 11 + 3).astype(np.uint8)
    for use_stream in (False, True):
        s = host.Stream("hip") if use_stream else None
        bufs = [host.Tensor("hip", F32, (n // 4,)) for _ in range(3)]
        back = np.zeros(n, np.uint8)
        host.backend_copy("hip", bufs[0].data_ptr, "hip", pattern.ctypes.data, "cpu", n, s)
        host.backend_copy("hip", bufs[1].data_ptr, "hip", bufs[0].data_ptr, "hip", n, s)
        host.backend_copy("hip", bufs[2].data_ptr, "hip", bufs[1].data_ptr, "hip", n, s)
        host.backend_copy("hip", back.ctypes.data, "cpu", bufs[2].data_ptr, "hip", n, s)
        if s is not None:
            s.synchronize()
        assert_bitwise(back, pattern, f"device round trip (stream={use_stream})")
        h2h = np.zeros(n, np.uint8)
        host.backend_copy("hip", h2h.ctypes.data, "cpu", pattern.ctypes.data, "cpu", n, s)
        if s is not None:
            s.synchronize()
        assert_bitwise(h2h, pattern, f"host-to-host copy (stream={use_stream})")
    with pytest.raises(host.FrameError, match="invalid_argument"):
        host.backend_copy("hip", 0, "hip", pattern.ctypes.data, "cpu", n)  # null destination


def test_backend_compile_of_an_op_without_kernel_is_unimplemented_with_its_name(dev):
    say("Backend::compile of an op with no hip kernel")
    text = ("%0 = graph_input() : float32[4]@hip:0\n"
            "%1 = frame_conformance_unsupported_op(%0) : float32[4]@hip:0\n"
            "graph_output(%1)\n")
    with pytest.raises(host.FrameError) as e:
        host.backend_compile(text, "hip")
    msg = str(e.value)
    assert msg.startswith("[unimplemented]"), msg
    assert "frame_conformance_unsupported_op" in msg, msg


# ---- the eager hop: every node through Backend::launch ------------------------------------------------------

_LINE = re.compile(r"^%(\d+) = ([A-Za-z_0-9]+)\(([^)]*)\)(?: (\{.*\}))? : (\S+)$")
_TYPE = re.compile(r"^([a-z0-9]+)\[([0-9,]*)\]@")
_DT = {"float32": F32, "float16": F16, "bfloat16": BF16}


def run_eager(text, inputs):
    """Runs the post-pipeline graph `text` node by node through Backend::launch (frame_launch), the way the
    reference's FallbackExecutable steps a graph; returns the graph outputs as numpy arrays."""
    vals, types, outs = {}, {}, []
    n_in = 0
    stream = host.Stream("hip")
    for line in text.strip().splitlines():
        if line.startswith("graph_output("):
            outs.append(int(line[len("graph_output(%"):-1]))
            continue
        m = _LINE.match(line)
        assert m, line
        vid, op, args, attrs, ty = int(m.group(1)), m.group(2), m.group(3), m.group(4), m.group(5)
        tm = _TYPE.match(ty)
        dtype, shape = _DT[tm.group(1)], tuple(int(d) for d in tm.group(2).split(",") if d)
        types[vid] = ty
        if op == "graph_input":
            vals[vid] = host.Tensor.from_numpy("hip", dtype, inputs[n_in])
            n_in += 1
            continue
        ids = [int(a.strip()[1:]) for a in args.split(",") if a.strip()]
        node = [f"%{i} = graph_input() : {types[a]}" for i, a in enumerate(ids)]
        node.append(f"%{len(ids)} = {op}({', '.join('%' + str(i) for i in range(len(ids)))})"
                    + (f" {attrs}" if attrs else "") + f" : {ty}")
        node.append(f"graph_output(%{len(ids)})")
        out = host.Tensor("hip", dtype, shape)
        host.launch("\n".join(node) + "\n", "hip", [vals[a] for a in ids], [out], stream)
        vals[vid] = out
    stream.synchronize()
    return [vals[o].numpy() for o in outs]


@pytest.mark.parametrize("which", ["c1", "c3_small", "c5_small"])
def test_eager_hop_node_by_node_matches_oracle(dev, which):
    if which == "c1":
        g, ins, dtype = graphs.mlp(batch=64, dtype=F32), graphs.mlp_inputs(batch=64, dtype=F32), F32
    elif which == "c3_small":
        cfg = dict(n=2, cin=64, h=12, w=12, cout=64, k=3)
        g, ins, dtype = graphs.conv(BF16, **cfg), graphs.conv_inputs(BF16, **cfg), BF16
    else:
        g, shapes = graphs.transformer_block(batch=2, seq=64, d_model=128, heads=4, ffn=512, dtype=BF16)
        ins, dtype = graphs.transformer_inputs(shapes, rows=128, d_model=128, dtype=BF16), BF16
    lowered = host.transform(g.text())  # the standard pipeline's graph, which FallbackExecutable would step
    say(f"eager hop {which}: {sum(1 for l in lowered.splitlines() if ' = ' in l)} nodes through Backend::launch")
    got = run_eager(lowered, ins)
    want = orc.run_graph_cpu(g.text().replace("@hip:0", "@cpu:0"), ins)
    for a, e in zip(got, want):
        assert_close(a, e, dtype, what=f"eager {which}")


@pytest.mark.parametrize("cfg", [dict(n=2, cin=64, h=14, w=14, cout=64, k=3, stride=1, pad=1),
                                 dict(n=2, cin=3, h=20, w=20, cout=16, k=7, stride=2, pad=3),
                                 dict(n=1, cin=96, h=9, w=11, cout=40, k=3, stride=2, pad=1)])
def test_eager_conv2d_takes_the_mfma_path(dev, cfg):
    """Backend::launch of conv2d on NCHW tensors: geometries the implicit-GEMM kernel takes run on MFMA through
    channels-last temporaries (the C8 pack for 3 channels)."""
    say(f"eager conv2d {cfg}")
    g = graphs.conv(BF16, device="hip", **cfg)
    ins = graphs.conv_inputs(BF16, n=cfg["n"], cin=cfg["cin"], h=cfg["h"], w=cfg["w"], cout=cfg["cout"], k=cfg["k"])
    text = g.text()
    conv_line = [l for l in text.splitlines() if "conv2d(" in l][0]
    node = "\n".join(text.splitlines()[:3] + [conv_line, "graph_output(%3)"]) + "\n"
    tm = _TYPE.match(conv_line.split(" : ")[1])
    out_shape = tuple(int(d) for d in tm.group(2).split(","))
    ts = [host.Tensor.from_numpy("hip", BF16, a) for a in ins]
    out = host.Tensor("hip", BF16, out_shape)
    host.launch(node, "hip", ts, [out])
    got = out.numpy()
    geom = (cfg["n"], cfg["cin"], cfg["h"], cfg["w"], cfg["cout"], cfg["k"], cfg["k"], cfg["stride"], cfg["stride"],
            cfg["pad"], cfg["pad"], 1)
    want = orc.conv2d(BF16, *ins, geom)
    assert_close(got, want, BF16, what=f"eager conv2d {cfg}")


# ---- allocator and arena lifetimes --------------------------------------------------------------------------

def test_run_with_allocated_outputs_keeps_device_memory_flat(dev):
    """run_with_allocated_outputs creates a stream per call (reference src/runtime/compile.cpp:180-220): the arena
    of each call's stream must not outlive the stream, and freed blocks must be reused, so 200 calls hold flat
    device memory."""
    for which, calls in (("c1", 200), ("c4_64px", 60)):
        if which == "c1":
            g, ins = graphs.mlp(batch=64, dtype=F32), graphs.mlp_inputs(batch=64, dtype=F32)
        else:
            g, specs = graphs.resnet18(batch=8, dtype=BF16, image=64)
            ins = graphs.resnet18_inputs(specs, batch=8, dtype=BF16, image=64)
        exe = host.compile(g, "hip")
        dev_ins = exe.upload_inputs(ins)
        first = None
        held = []
        for i in range(calls):
            (out,) = exe.run(dev_ins)
            if i == 0:
                first = out
            else:
                assert_bitwise(out, first, f"{which} call {i}")
            st = host.allocator_stats()
            held.append(st["live"] + st["cached"] + st["pending"])
        say(f"{which}: bytes held by the allocator after calls 10 / {calls}: {held[9]} / {held[-1]}; {host.allocator_stats()}")
        assert held[-1] <= held[9], (which, held[9], held[-1])


def test_freed_block_is_not_reused_while_queued_work_writes_it(dev):
    """An output freed while the kernels writing it are still queued: the next allocation of that size must not
    receive the block before those kernels finish, so a synchronous upload into the new tensor survives. The wait
    is on the block's own fence events, not a device-wide synchronisation."""
    g = graphs.gemm(4096, BF16)
    exe = host.compile(g, "hip")
    ins = exe.upload_inputs(graphs.gemm_inputs(4096, BF16))
    stream = host.Stream("hip")
    pattern = synth.to_storage(np.full((4096, 4096), 0.5, np.float32), BF16)
    syncs0 = host.allocator_stats()["device_syncs"]
    for trial in range(3):
        (t1,) = exe.alloc_outputs()
        addr = t1.data_ptr
        for _ in range(4):  # ~0.5 ms of GEMMs writing t1
            exe.run_tensors(ins, [t1], stream)
        del t1  # freed while the GEMMs are queued
        t2 = host.Tensor.from_numpy("hip", BF16, pattern)  # same size class; synchronous null-stream upload
        stream.synchronize()
        assert_bitwise(t2.numpy(), pattern, f"trial {trial}: block reused under queued writes (t1 {addr:#x}, "
                                            f"t2 {t2.data_ptr:#x})")
        del t2
    st = host.allocator_stats()
    say(f"allocator after the trials: {st}")
    assert st["device_syncs"] == syncs0, st


def test_per_stream_arenas_are_bounded(dev):
    """An executable run on many live streams keeps at most a bounded number of arenas; arenas of destroyed
    streams are dropped."""
    g = graphs.mlp(batch=64, dtype=F32)
    exe = host.compile(g, "hip")
    ins = exe.upload_inputs(graphs.mlp_inputs(batch=64, dtype=F32))
    outs = exe.alloc_outputs()
    streams = [host.Stream("hip") for _ in range(12)]
    for s in streams:
        exe.run_tensors(ins, outs, s)
        s.synchronize()
    live_many = host.allocator_stats()["live"]
    del streams
    for _ in range(3):
        s = host.Stream("hip")
        exe.run_tensors(ins, outs, s)
        s.synchronize()
        del s
    live_after = host.allocator_stats()["live"]
    say(f"live bytes with 12 streams: {live_many}; after they are destroyed: {live_after}")
    assert live_after < live_many


def test_run_repeat_rotates_input_sets_like_single_runs(dev):
    """frame_executable_run_repeat (the benchmark's native timed loop): run i reads input set i % n; after 5 runs
    over 2 sets the outputs are those of a single run on set 0, bit for bit, and match the oracle."""
    g = graphs.mlp(batch=64, dtype=F32)
    exe = host.compile(g, "hip")
    sets_np = [graphs.mlp_inputs(batch=64, dtype=F32, seed=s) for s in (1, 2)]
    sets = [exe.upload_inputs(s) for s in sets_np]
    stream = host.Stream("hip")
    outs = exe.alloc_outputs()
    exe.run_repeat(sets, outs, stream, 5)
    stream.synchronize()
    got = outs[0].numpy()
    single = exe.alloc_outputs()
    exe.run_tensors(sets[0], single, stream)
    stream.synchronize()
    assert_bitwise(got, single[0].numpy(), "run_repeat vs a single run")
    (want,) = orc.run_graph_cpu(graphs.mlp(batch=64, dtype=F32, device="cpu"), sets_np[0])
    assert_close(got, want, F32, what="run_repeat vs oracle")
    exe.run_repeat(sets, outs, stream, 0)  # zero runs: nothing enqueued
    stream.synchronize()
    assert_bitwise(outs[0].numpy(), got, "after zero runs")

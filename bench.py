"""Benchmark of the `hip` backend's compiled-graph hot path on one MI355X.

Workload (the dense GEMM sweep, at its largest size): C = A·B, row-major
A[4096,4096]·B[4096,4096], bfloat16 inputs, fp32 accumulation, bfloat16 output; entries U(-1,1) from the
build's seeded generator. One step = one forward pass of that graph on inputs already resident in HBM.

Prints ONE JSON line with the metric (TFLOP/s), the dominant kernel's roofline fraction (its average duration
measured with HIP events on the stream it runs on) and a CPU baseline: the reference's own CPU backend
(oracle/_ref, single-threaded) timed on a bounded row-sample of the same GEMM on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(REPO, "frame-public_amd"), os.path.join(REPO, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

import numpy as np  # noqa: E402

PEAK_BF16_TFLOPS = 2516.6  # dense bf16 MFMA, 256 CU x 2.4 GHz x 4096 FLOP/clk/CU
PEAK_F32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
GRAPH_SETTLE_MS = 200.0  # untimed wall time each secondary measurement runs before its timed region

N = 4096
F32, BF16 = 0, 3


def gemm_flops(m, n, k):
    return 2.0 * m * n * k


class _NativeStream:
    """The hipStream_t under a hal::Stream, for HIP events recorded on the stream the kernels run on."""

    def __init__(self, ptr):
        self.ptr = ptr


def gemm_operands(data: str):
    """The headline's operands: U(-1,1) (the configuration's data), or all zeros / all ones for the
    data-dependence check of the engine clock (same kernel, same work, less switching)."""
    from frame_hip import graphs, synth

    if data == "uniform":
        return graphs.gemm_inputs(N, BF16)
    value = 0.0 if data == "zeros" else 1.0
    return [synth.to_storage(np.full((N, N), value, np.float32), BF16) for _ in range(2)]


def run_gpu(steps: int, warmup: int, data: str = "uniform", settle_ms: float = 300.0):
    """Times `steps` runs of the compiled GEMM graph (runtime::compile(graph, "hip") -> Executable::run) on one
    persistent stream, inputs and outputs resident in HBM.

    After the `warmup` steps, further untimed steps run until `settle_ms` of wall time has passed since the
    first one: the MI355X raises its engine clock over the first ~10 ms of sustained MFMA load (50 back-to-back
    launches of this GEMM time ~15 % slower from a cold start than the same 50 a few milliseconds later), so a
    few warmup steps alone time the clock ramp instead of the kernel. Returns (ms per step, wall seconds of the
    timed region, settle steps run)."""
    from frame_hip import abi, graphs, host

    g = graphs.gemm(N, BF16, device="hip")
    exe = host.compile(g, "hip")
    ins = exe.upload_inputs(gemm_operands(data))
    outs = exe.alloc_outputs()
    stream = host.Stream("hip")
    native = _NativeStream(stream.native)
    start, stop = abi.Event(), abi.Event()
    t_start = time.perf_counter()
    for _ in range(warmup):
        exe.run_tensors(ins, outs, stream)
    stream.synchronize()
    settle = 0
    while (time.perf_counter() - t_start) * 1e3 < settle_ms:
        for _ in range(20):
            exe.run_tensors(ins, outs, stream)
        stream.synchronize()
        settle += 20
    abi.check(abi.lib().fh_device_synchronize())
    t0 = time.perf_counter()
    start.record(native)
    exe.run_repeat([ins], outs, stream, steps)  # the K timed runs, issued from native code
    stop.record(native)
    stop.synchronize()
    stream.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_ms(stop) / steps
    return ms, wall, settle


TRAFFIC_SUMMARY = os.path.join(REPO, "profiles", "gemm16_bf16_4096_hbm_traffic.md")


def measured_traffic():
    """HBM bytes per launch of the GEMM kernel, from the committed FETCH_SIZE / WRITE_SIZE counter passes
    (scaled by the same counters on a plain copy of known size); None where no such summary exists."""
    try:
        with open(TRAFFIC_SUMMARY) as f:
            m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", f.read(), re.M)
    except OSError:
        return None
    return int(m.group(1)) if m else None


def copy_calibration(mib: int, reps: int):
    """Launches copy2d_kernel (fh_copy2d, one 16-byte load and store per lane) over `mib` MiB, `reps` times:
    the known-size copy that scales the FETCH_SIZE / WRITE_SIZE counters of the traffic passes."""
    from frame_hip import abi

    nbytes = mib << 20
    src, dst = abi.DeviceBuffer(nbytes), abi.DeviceBuffer(nbytes)
    abi.check(abi.lib().fh_fill(src.ptr, 4, 0x3F800000, nbytes // 4, None), "fh_fill")
    for _ in range(reps):
        abi.check(abi.lib().fh_copy2d(dst.ptr, nbytes, src.ptr, nbytes, nbytes, 1, None), "fh_copy2d")
    abi.check(abi.lib().fh_device_synchronize(), "fh_device_synchronize")
    print(json.dumps({"copy_calibration_bytes": nbytes, "launches": reps}), flush=True)


# ---- secondary measurements of the same metric (GEMM/Conv2d TFLOP/s, fused-op GB/s, graph latency) --

def _time_graph(graph_text, input_sets, steps, warmup, settle_ms=GRAPH_SETTLE_MS):
    """ms per Executable::run of the compiled graph, rotating over input_sets (lists of numpy arrays), HIP events
    on the executable's own stream. After the warm-up runs the graph keeps running, untimed, for settle_ms of
    wall time, so the timed runs see the settled engine clock rather than its ramp from idle (a short graph
    such as C1 otherwise measures up to 2.5x its settled time on a cold GPU)."""
    from frame_hip import abi, host

    exe = host.compile(graph_text, "hip")
    sets = [exe.upload_inputs(s) for s in input_sets]
    outs = exe.alloc_outputs()
    stream = host.Stream("hip")
    native = _NativeStream(stream.native)
    start, stop = abi.Event(), abi.Event()
    for i in range(warmup):
        exe.run_tensors(sets[i % len(sets)], outs, stream)
    stream.synchronize()
    t_end = time.perf_counter() + settle_ms * 1e-3
    while time.perf_counter() < t_end:
        exe.run_repeat(sets, outs, stream, 16)
        stream.synchronize()
    stream.synchronize()
    start.record(native)
    # the timed runs are issued from native code (frame_executable_run_repeat), as the reference's google-benchmark
    # loops call Executable::run from C++ (benchmarks/bench_matmul.cpp): a Python loop costs more per run than a
    # short graph's kernels (LayerNorm's one 4 us launch) and would time the interpreter instead
    exe.run_repeat(sets, outs, stream, steps)
    stop.record(native)
    stop.synchronize()
    return start.elapsed_ms(stop) / steps


def _time_train_step(fwd_text, n_params, inputs, lr, steps, warmup):
    """ms per training step of the forward graph `fwd_text` whose inputs 1..n_params are the parameters: the
    backward graph (forward outputs + gradients, compiler::build_backward_graph) then the SGD update graph,
    parameters ping-ponging between two buffer sets on one stream; HIP events around `steps` steps."""
    from frame_hip import abi, host

    wrt = list(range(1, n_params + 1))
    train = host.compile(host.backward(fwd_text, 0, wrt), "hip")
    sgd = host.compile(host.sgd_update(fwd_text, wrt, lr), "hip")
    ins = train.upload_inputs(inputs)
    outs = train.alloc_outputs()
    params = [ins[1:n_params + 1], sgd.alloc_outputs()]
    stream = host.Stream("hip")
    native = _NativeStream(stream.native)
    start, stop = abi.Event(), abi.Event()

    def step(i):
        cur, nxt = params[i % 2], params[(i + 1) % 2]
        train.run_tensors([ins[0]] + cur + ins[n_params + 1:], outs, stream)
        sgd.run_tensors(cur + outs[1:], nxt, stream)

    for i in range(warmup):
        step(i)
    stream.synchronize()
    t_end = time.perf_counter() + GRAPH_SETTLE_MS * 1e-3  # settled clock, as in _time_graph
    while time.perf_counter() < t_end:
        step(warmup)
        warmup += 1
        stream.synchronize()
    start.record(native)
    for i in range(steps):
        step(warmup + i)
    stop.record(native)
    stop.synchronize()
    return start.elapsed_ms(stop) / steps


def extras(steps, only=None):
    """Each entry: the config, its work, and the measured rate; failures are reported, not raised.
    `only` names one entry to run by itself (for per-workload profiles)."""
    from frame_hip import graphs, synth

    out = {}

    def guard(name, fn):
        if only is not None and name != only:
            return
        try:
            out[name] = fn()
        except Exception as e:  # a secondary measurement must not cost the bench line
            out[name] = {"error": f"{type(e).__name__}: {e}"}

    def fused():
        # C4's residual add;relu at layer-1 shape, bf16; 8 input sets (616 MB) so every run reads from HBM
        shape = (64, 64, 56, 56)
        g = graphs.Graph("hip")
        x, y = g.input(BF16, shape), g.input(BF16, shape)
        g.output(g.relu(g.add(x, y)))
        sets = [[synth.tensor(900 + 2 * i, shape, BF16), synth.tensor(901 + 2 * i, shape, BF16)] for i in range(8)]
        ms = _time_graph(g.text(), sets, max(steps, 40), 8)
        by = 3 * int(np.prod(shape)) * 2
        return {"workload": "fused add;relu bf16 [64,64,56,56], cold (8 rotating input sets)", "us": round(ms * 1e3, 2),
                "GB/s": round(by / (ms * 1e-3) / 1e9, 1), "frac_hbm": round(by / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}

    def rows_op(kind):
        # C5's row reductions as standalone ops: softmax over the [8*16*512, 512] per-head score rows, LayerNorm
        # over the [4096, 1024] activations; bf16, 8 rotating input sets so every run reads from HBM
        g = graphs.Graph("hip")
        if kind == "softmax":
            shape = (65536, 512)
            x = g.input(BF16, shape)
            g.output(g.softmax(x))
            sets = [[synth.tensor(920 + i, shape, BF16, "normal", 2.0)] for i in range(8)]
            by = 2 * int(np.prod(shape)) * 2
        else:
            shape = (4096, 1024)
            x, ga, be = g.input(BF16, shape), g.input(BF16, (1024,)), g.input(BF16, (1024,))
            g.output(g.layer_norm(x, ga, be))
            sets = [[synth.tensor(930 + i, shape, BF16), synth.tensor(940, (1024,), BF16), synth.tensor(941, (1024,), BF16)]
                    for i in range(8)]
            by = 2 * int(np.prod(shape)) * 2 + 2 * 1024 * 2
        ms = _time_graph(g.text(), sets, max(steps, 40), 8)
        # the copy floor at the same bytes: relu(x) of the same shape (one read, one write) through the fused
        # elementwise kernel, timed the same way
        gc = graphs.Graph("hip")
        gc.output(gc.relu(gc.input(BF16, shape)))
        copy_ms = _time_graph(gc.text(), [s_[:1] for s_ in sets], max(steps, 40), 8)
        return {"workload": f"{kind} bf16 {list(shape)}, cold (8 rotating input sets)", "us": round(ms * 1e3, 2),
                "GB/s": round(by / (ms * 1e-3) / 1e9, 1), "frac_hbm": round(by / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                "copy_us": round(copy_ms * 1e3, 2)}

    def conv(dtype):
        flops = 2 * 32 * 64 * 56 * 56 * 64 * 9
        ms = _time_graph(graphs.conv(dtype).text(), [graphs.conv_inputs(dtype)], max(3, steps // 5), 2)
        tf = flops / (ms * 1e-3) / 1e12
        peak = PEAK_BF16_TFLOPS if dtype == BF16 else PEAK_F32_TFLOPS
        return {"workload": f"C3 conv2d+bias+relu {'bf16' if dtype == BF16 else 'f32'} [32,64,56,56]*[64,64,3,3], whole compiled graph",
                "us": round(ms * 1e3, 1), "TFLOP/s": round(tf, 1), "frac_mfma": round(tf / peak, 4)}

    def gemm(n, dtype):
        ms = _time_graph(graphs.gemm(n, dtype).text(), [graphs.gemm_inputs(n, dtype)], max(10, steps // 2), 3)
        tf = gemm_flops(n, n, n) / (ms * 1e-3) / 1e12
        peak = PEAK_BF16_TFLOPS if dtype == BF16 else PEAK_F32_TFLOPS
        return {"TFLOP/s": round(tf, 1), "frac_mfma": round(tf / peak, 4), "us": round(ms * 1e3, 1)}

    def mlp():
        ms = _time_graph(graphs.mlp(64, F32).text(), [graphs.mlp_inputs(64, F32)], max(50, steps), 10)
        return {"workload": "C1 MLP f32 batch 64, compiled graph", "us": round(ms * 1e3, 1)}

    def resnet():
        g, specs = graphs.resnet18(batch=64, dtype=BF16)
        ms = _time_graph(g.text(), [graphs.resnet18_inputs(specs, batch=64, dtype=BF16)], max(5, steps // 5), 2)
        return {"workload": "C4 ResNet-18 bf16 batch 64 224px, compiled graph", "ms": round(ms, 3),
                "TFLOP/s": round(232.2e9 / (ms * 1e-3) / 1e12, 1)}

    def transformer():
        g, shapes = graphs.transformer_block(dtype=BF16)
        ms = _time_graph(g.text(), [graphs.transformer_inputs(shapes, dtype=BF16)], max(5, steps // 5), 2)
        return {"workload": "C5 transformer block bf16 8x512x1024, 16 heads, FFN 4096, compiled graph", "ms": round(ms, 3),
                "TFLOP/s": round(111.67e9 / (ms * 1e-3) / 1e12, 1)}

    def mlp_train():
        g = graphs.mlp_train(batch=64, dtype=F32)
        ms = _time_train_step(g.text(), 4, graphs.mlp_train_inputs(batch=64, dtype=F32), 0.01, max(50, steps), 10)
        return {"workload": "C1 MLP f32 batch 64 training step (mse_loss, backward graph + SGD update graph)",
                "us": round(ms * 1e3, 1)}

    def resnet_train():
        g, specs = graphs.resnet18(batch=64, dtype=BF16, train=True)
        ins = graphs.resnet18_inputs(specs, batch=64, dtype=BF16) + [synth.tensor(499, (64, 1000), BF16, "normal")]
        ms = _time_train_step(g.text(), len(specs), ins, 1e-3, max(2, steps // 25), 1)
        return {"workload": "C4 ResNet-18 bf16 batch 64 224px training step (mse_loss, backward + SGD graphs)",
                "ms": round(ms, 3), "TFLOP/s": round(3 * 232.2e9 / (ms * 1e-3) / 1e12, 1)}

    def conv_grads(dtype):
        # C3's conv: both gradients at [32,64,56,56] * [64,64,3,3], 7.399 GFLOP each
        geo = dict(stride=[1, 1], padding=[1, 1], groups=1)
        xs, ws = (32, 64, 56, 56), (64, 64, 3, 3)
        res = {}
        for name, ins_s, out_s, extra in [("grad_input", [xs, ws], xs, {"input_shape": graphs.Shape(xs)}),
                                          ("grad_filter", [xs, xs], ws, {"filter_shape": graphs.Shape(ws)})]:
            g = graphs.Graph("hip")
            vals = [g.input(dtype, sh) for sh in ins_s]
            g.output(g.op(f"conv2d_{name}_internal", vals, out_s, dict(geo, **extra)))
            ins = [synth.tensor(700 + i, sh, dtype, "normal") for i, sh in enumerate(ins_s)]
            ms = _time_graph(g.text(), [ins], max(3, steps // 10), 1)
            res[name] = {"us": round(ms * 1e3, 1), "TFLOP/s": round(7.399e9 / (ms * 1e-3) / 1e12, 1)}
        res["workload"] = f"C3 conv gradients {'bf16' if dtype == BF16 else 'f32'} [32,64,56,56]*[64,64,3,3]"
        return res

    def graph_replay():
        # eager step launches against the captured-hipGraph replay (FRAME_HIP_GRAPHS=1) of the same executable
        cfgs = {"c1_mlp": (graphs.mlp(64, F32).text(), [graphs.mlp_inputs(64, F32)], 200, 20)}
        g4, specs = graphs.resnet18(batch=64, dtype=BF16)
        cfgs["c4_resnet18"] = (g4.text(), [graphs.resnet18_inputs(specs, batch=64, dtype=BF16)], 20, 5)
        g5, shapes = graphs.transformer_block(dtype=BF16)
        cfgs["c5_transformer"] = (g5.text(), [graphs.transformer_inputs(shapes, dtype=BF16)], 40, 5)
        res = {}
        for name, (text, sets, n, w) in cfgs.items():
            row = {}
            for mode in ("eager", "replay", "eager_again"):
                if mode == "replay":
                    os.environ["FRAME_HIP_GRAPHS"] = "1"
                else:
                    os.environ.pop("FRAME_HIP_GRAPHS", None)
                row[mode + "_us"] = round(_time_graph(text, sets, n, w) * 1e3, 1)
            os.environ.pop("FRAME_HIP_GRAPHS", None)
            res[name] = row
        return res

    def cpu_baselines():
        # the reference CPU backend (oracle/_ref, one thread) on a bounded sample of each configuration, scaled to
        # the configuration (every op here computes each image / sequence independently, so the scale is exact)
        import oracle_lib as orc

        if not orc.ref_available():
            return {"error": "oracle/_ref is not built"}
        res = {"cores": 1, "nproc": os.cpu_count(), "cpu_model": _cpu_model()}

        def timed(text, ins, out_specs, reps=1):
            t0 = time.perf_counter()
            for _ in range(reps):
                orc.ref_run_graph(text.replace("@hip:0", "@cpu:0"), ins, out_specs)
            return (time.perf_counter() - t0) / reps

        t = timed(graphs.mlp(64, F32).text(), graphs.mlp_inputs(64, F32), [((64, 10), np.float32)], reps=20)
        res["c1_mlp"] = {"sample": "the whole batch-64 forward, 20 runs", "ms": round(t * 1e3, 3)}
        t = timed(graphs.conv(BF16, n=1).text(), graphs.conv_inputs(BF16, n=1), [((1, 64, 56, 56), np.uint16)])
        res["conv_c3_bf16"] = {"sample": "image 1 of 32", "ms": round(t * 32 * 1e3, 1),
                               "TFLOP/s": round(7.399e9 / (t * 32) / 1e12, 6)}
        g, specs = graphs.resnet18(batch=1, dtype=BF16)
        t = timed(g.text(), graphs.resnet18_inputs(specs, batch=1, dtype=BF16), [((1, 1000), np.uint16)])
        res["c4_resnet18"] = {"sample": "image 1 of 64", "ms": round(t * 64 * 1e3, 1),
                              "TFLOP/s": round(232.2e9 / (t * 64) / 1e12, 6)}
        g, shapes = graphs.transformer_block(batch=1, dtype=BF16, act="relu")
        t = timed(g.text(), graphs.transformer_inputs(shapes, rows=512, dtype=BF16), [((512, 1024), np.uint16)])
        res["c5_transformer"] = {"sample": "sequence 1 of 8, relu in place of gelu (the reference has no gelu op)",
                                 "ms": round(t * 8 * 1e3, 1), "TFLOP/s": round(111.67e9 / (t * 8) / 1e12, 6)}
        return res

    def vendor(shapes):
        # Yardstick only, on request: the vendor GEMM (hipBLASLt through torch.matmul, and torch.addmm with a full-size
        # C as the graphs' bias inputs are) on bf16 U(-1,1) operands, after the same kind of settle; nothing of this
        # repository runs in it
        import torch

        torch.manual_seed(0)
        res = {}
        for (m, n, k) in shapes:
            a = (torch.rand(m, k, device="cuda") * 2 - 1).to(torch.bfloat16)
            b = (torch.rand(k, n, device="cuda") * 2 - 1).to(torch.bfloat16)
            c = (torch.rand(m, n, device="cuda") * 2 - 1).to(torch.bfloat16)
            entry = {}
            for name, fn in (("matmul", lambda: a @ b), ("addmm", lambda: torch.addmm(c, a, b))):
                fn()
                torch.cuda.synchronize()
                t_end = time.perf_counter() + GRAPH_SETTLE_MS * 1e-3
                while time.perf_counter() < t_end:
                    for _ in range(10):
                        fn()
                    torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(max(steps, 20)):
                    fn()
                e1.record()
                e1.synchronize()
                us = e0.elapsed_time(e1) / max(steps, 20) * 1e3
                entry[name] = {"us": round(us, 2), "TFLOP/s": round(gemm_flops(m, n, k) / (us * 1e-6) / 1e12, 1)}
            res[f"{m}x{n}x{k}"] = entry
        return res

    if only is not None:
        guard("graph_replay", graph_replay)
        guard("cpu_baselines", cpu_baselines)
        guard("vendor_gemm_4096", lambda: vendor([(4096, 4096, 4096)]))
        guard("vendor_gemm_c5", lambda: vendor([(4096, 3072, 1024), (4096, 1024, 1024), (4096, 4096, 1024),
                                                (4096, 1024, 4096)]))
    guard("fused_elementwise", fused)
    guard("softmax_c5", lambda: rows_op("softmax"))
    guard("layer_norm_c5", lambda: rows_op("layer_norm"))
    guard("conv_c3_bf16", lambda: conv(BF16))
    guard("conv_c3_f32", lambda: conv(F32))
    for n in (1024, 2048):
        guard(f"gemm_bf16_{n}", lambda n=n: gemm(n, BF16))
    for n in (1024, 2048, 4096):
        guard(f"gemm_f32_{n}", lambda n=n: gemm(n, F32))
    guard("c1_mlp_latency", mlp)
    guard("c4_resnet18", resnet)
    guard("c5_transformer", transformer)
    guard("c1_mlp_train_step", mlp_train)
    guard("conv_c3_grads_bf16", lambda: conv_grads(BF16))
    guard("c4_resnet18_train_step", resnet_train)
    return out


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(rows: int):
    """Reference CPU backend (single thread) on rows x 4096 x 4096 of the same GEMM."""
    import oracle_lib as orc
    from frame_hip import synth

    a = synth.tensor(31, (N, N), BF16, "uniform")[:rows].copy()
    b = synth.tensor(32, (N, N), BF16, "uniform")
    if orc.ref_available():
        text = (f"%0 = graph_input() : bfloat16[{rows},{N}]@cpu:0\n"
                f"%1 = graph_input() : bfloat16[{N},{N}]@cpu:0\n"
                f"%2 = matmul(%0, %1) : bfloat16[{rows},{N}]@cpu:0\n"
                f"graph_output(%2)\n")
        t0 = time.perf_counter()
        orc.ref_run_graph(text, [a, b], [((rows, N), np.uint16)])
        dt = time.perf_counter() - t0
        kind = "reference"
    else:
        t0 = time.perf_counter()
        orc.matmul(BF16, a, b)
        dt = time.perf_counter() - t0
        kind = "port"
    return {"value": gemm_flops(rows, N, N) / dt / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": kind,
            "sample": f"{rows} of {N} output rows of the bf16 {N}^3 GEMM ({gemm_flops(rows, N, N) / 1e9:.1f} GFLOP), "
                      f"{dt:.1f} s single-threaded"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--settle-ms", type=float, default=300.0,
                    help="untimed steps after the warmup until this much wall time has passed (engine clock ramp)")
    ap.add_argument("--cpu-rows", type=int, default=128)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="only the headline GEMM (and the CPU baseline)")
    ap.add_argument("--gemm-data", choices=["uniform", "zeros", "ones"], default="uniform",
                    help="headline operands; anything but the default (U(-1,1), the configuration's data) is a "
                         "diagnostic of data-dependent clocks and is labelled as such in the output")
    ap.add_argument("--only", default=None,
                    help="run just this secondary measurement (e.g. c5_transformer) and print it, no headline")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="only run the known-size copy used to scale HBM traffic counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one MI355X only (no multi-GPU path); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration_mib > 0:
        copy_calibration(args.copy_calibration_mib, args.steps)
        return
    if args.only:
        print(json.dumps({args.only: extras(args.steps, args.only).get(args.only, {"error": "no such entry"})}), flush=True)
        return

    ms, wall, settle = run_gpu(args.steps, args.warmup, args.gemm_data, args.settle_ms)
    tflops = gemm_flops(N, N, N) / (ms * 1e-3) / 1e12
    line = {
        "metric": "GEMM/Conv2d TFLOP/s & % MFMA peak; fused-op GB/s; compiled-graph fwd latency",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"ms": args.settle_ms, "untimed_steps": settle},
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic" if args.gemm_data == "uniform" else f"synthetic, diagnostic all-{args.gemm_data} operands",
        "config": {"workload": "dense GEMM C=A·B, M=N=K=4096, bf16 in/out, fp32 accumulate (configs[1])",
                   "M": N, "N": N, "K": N},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_BF16_TFLOPS, 4), "traffic": measured_traffic()},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.cpu_rows)
    if not args.no_extras:
        line["extras"] = extras(args.steps)
        line["extras_settle_ms"] = GRAPH_SETTLE_MS
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

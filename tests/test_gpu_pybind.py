"""Python -> hip through the pybind11 module frame_hip_py, the way the reference's Python surface runs a graph
(python/src/bind_runtime.cpp:33-43: compile(graph, backend) then Executable.run(inputs), i.e.
runtime::run_with_allocated_outputs), and weights imported from ONNX (bind_interop.cpp:38-74): C1's MLP on hip
equals the ctypes C-API path bit for bit and the oracle within the fp32 rule; weights saved to ONNX, loaded
back and uploaded give the same outputs bit for bit (the reference's train-save-import-infer check,
tests/cpp/interop/test_onnx_weights.cpp:372)."""
import os
import sys

import numpy as np
import pytest

import oracle_lib as orc
from frame_hip import graphs, host
from tolerance import assert_bitwise, assert_close

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "frame-public_amd", "lib")
if LIB not in sys.path:
    sys.path.insert(0, LIB)
import frame_hip_py as fp  # noqa: E402

pytestmark = pytest.mark.gpu
F32 = 0


def test_compile_and_run_through_pybind(tmp_path):
    print("[case] C1 MLP through frame_hip_py", flush=True)
    g = graphs.mlp(batch=64, dtype=F32, device="hip")
    ins = graphs.mlp_inputs(batch=64, dtype=F32)
    exe = fp.compile(g.text(), "hip")
    (out,) = exe.run([fp.Tensor.from_numpy("hip", F32, a) for a in ins])
    assert out.backend == "hip" and tuple(out.shape) == (64, 10)
    got = out.numpy()
    assert_bitwise(got, host.compile(g, "hip").run(ins)[0], "pybind vs C API")
    orc.load_cpu_backend()
    (want,) = orc.run_graph_cpu(g.text().replace("@hip:0", "@cpu:0"), ins)
    assert_close(got, want, F32, what="C1 through pybind")

    # weights through ONNX: x stays, W1 b1 W2 b2 are saved, loaded and uploaded
    path = str(tmp_path / "mlp.onnx")
    names = ["w1", "b1", "w2", "b2"]
    fp.save_onnx_weights(path, {n: fp.Tensor.from_numpy("cpu", F32, a) for n, a in zip(names, ins[1:])})
    loaded = fp.load_onnx_weights(path)
    assert list(loaded) == names
    dev = [fp.Tensor.from_numpy("hip", F32, ins[0])] + [fp.Tensor.from_numpy("hip", F32, loaded[n].numpy()) for n in names]
    (again,) = exe.run(dev)
    assert_bitwise(again.numpy(), got, "weights imported from ONNX")

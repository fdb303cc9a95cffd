"""The pybind11 module frame_hip_py (reference surface: python/src/bind_runtime.cpp:33-56,
bind_interop.cpp:38-74), host-only parts: it imports from the in-tree build, its ONNX functions write the same
bytes as the C API (and so as the reference build) and load them back, and compiling for `hip` without a device
fails with a Python exception rather than a crash."""
import os
import sys

import numpy as np
import pytest

from frame_hip import host, synth

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "frame-public_amd", "lib")
if LIB not in sys.path:
    sys.path.insert(0, LIB)
import frame_hip_py as fp  # noqa: E402

F32, BF16 = 0, 3


def test_onnx_through_pybind_matches_the_c_api(tmp_path):
    w = {"w": (F32, synth.tensor(3, (16, 8), F32, "normal")), "b": (BF16, synth.tensor(4, (8,), BF16, "normal"))}
    ours = str(tmp_path / "py.onnx")
    fp.save_onnx_weights(ours, {k: fp.Tensor.from_numpy("cpu", dt, a) for k, (dt, a) in w.items()})
    capi = str(tmp_path / "capi.onnx")
    host.save_onnx_weights(capi, w)
    assert open(ours, "rb").read() == open(capi, "rb").read()
    got = fp.load_onnx_weights(capi)
    assert list(got) == ["w", "b"]
    for k, (dt, a) in w.items():
        assert got[k].dtype == dt and got[k].backend == "cpu" and tuple(got[k].shape) == a.shape
        assert got[k].numpy().tobytes() == a.tobytes()
    with pytest.raises(KeyError):
        fp.load_onnx_weights(str(tmp_path / "missing.onnx"))


@pytest.mark.skipif(host.device_count("hip") > 0, reason="a hip device is present")
def test_compile_without_a_device_raises():
    text = "%0 = graph_input() : float32[4]@hip:0\n%1 = relu(%0) : float32[4]@hip:0\ngraph_output(%1)\n"
    with pytest.raises(ValueError):
        fp.compile(text, "hip")


@pytest.mark.parametrize("code,exc", [(1, ValueError), (2, KeyError), (3, RuntimeError), (4, NotImplementedError),
                                      (5, MemoryError), (6, RuntimeError), (7, RuntimeError)])
def test_status_codes_map_to_the_reference_exceptions(code, exc):
    """Every frame::ErrorCode becomes the exception type of the reference binding (python/src/translate_status.cpp:
    29-47: kInvalidArgument ValueError, kNotFound KeyError, kUnimplemented NotImplementedError, kOutOfMemory
    MemoryError, the rest RuntimeError) with the status message verbatim."""
    msg = f"status message {code}: op 'x' kernel failed"
    with pytest.raises(exc) as info:
        fp._raise_status(code, msg)
    assert type(info.value) is exc
    text = info.value.args[0] if info.value.args else ""
    assert text == msg, (text, msg)
    fp._raise_status(0, "ok")  # kOk raises nothing

"""ctypes binding of the Frame host library's C API (include/frame_capi.h, lib/libframe.so).

This is how Python reaches Frame's compiled-graph path: IR text -> runtime::compile(graph, backend) ->
Executable::run, the same surface the reference exposes through pybind11 (reference:
python/src/bind_runtime.cpp:30-56). Loading fails loudly when the in-tree library is missing.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_int32, c_int64, c_size_t, c_void_p

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST_LIB = os.path.join(PKG_DIR, "lib", "libframe.so")

F32, F16, BF16 = 0, 2, 3
_NP = {0: np.float32, 1: np.float64, 2: np.uint16, 3: np.uint16, 4: np.int8, 5: np.int16, 6: np.int32, 7: np.int64,
       8: np.uint8, 9: np.bool_}
_ITEM = {0: 4, 1: 8, 2: 2, 3: 2, 4: 1, 5: 2, 6: 4, 7: 8, 8: 1, 9: 1}
CODES = {"ok": 0, "invalid_argument": 1, "not_found": 2, "already_exists": 3, "unimplemented": 4,
         "out_of_memory": 5, "internal": 6, "device_error": 7}


class FrameError(RuntimeError):
    def __init__(self, code: int, message: str):
        names = {v: k for k, v in CODES.items()}
        super().__init__(f"[{names.get(code, code)}] {message}")
        self.code = code


_lib = None
_SIGS = {
    "frame_last_error": (c_char_p, []),
    "frame_backends": (c_int32, [c_void_p, c_int64, POINTER(c_int64)]),
    "frame_device_count": (c_int32, [c_char_p, POINTER(c_int32)]),
    "frame_tensor_empty": (c_int32, [c_char_p, c_int32, c_int32, POINTER(c_int64), c_int32, POINTER(c_void_p)]),
    "frame_hip_run_tapped": (c_int32, [c_void_p, POINTER(c_void_p), c_int32, POINTER(c_void_p), c_int32, c_void_p, c_int32,
                                       POINTER(c_int32), POINTER(c_int32), POINTER(c_void_p), POINTER(c_int64)]),
    "frame_hip_executable_steps": (c_int32, [c_void_p, c_char_p, c_int64, POINTER(c_int64)]),
    "frame_tensor_empty_at": (c_int32, [c_char_p, c_int32, c_int32, POINTER(c_int64), c_int32, c_int64,
                                        POINTER(c_void_p)]),
    "frame_tensor_free": (None, [c_void_p]),
    "frame_tensor_data": (c_void_p, [c_void_p]),
    "frame_tensor_nbytes": (c_int64, [c_void_p]),
    "frame_tensor_upload": (c_int32, [c_void_p, c_void_p, c_size_t]),
    "frame_tensor_download": (c_int32, [c_void_p, c_void_p, c_size_t]),
    "frame_stream_create": (c_int32, [c_char_p, c_int32, POINTER(c_void_p)]),
    "frame_stream_destroy": (None, [c_void_p]),
    "frame_stream_synchronize": (c_int32, [c_void_p]),
    "frame_stream_native": (c_void_p, [c_void_p]),
    "frame_event_create": (c_int32, [c_char_p, c_int32, POINTER(c_void_p)]),
    "frame_event_destroy": (None, [c_void_p]),
    "frame_event_record": (c_int32, [c_void_p, c_void_p]),
    "frame_event_synchronize": (c_int32, [c_void_p]),
    "frame_compile": (c_int32, [c_char_p, c_char_p, c_int32, POINTER(c_void_p)]),
    "frame_executable_free": (None, [c_void_p]),
    "frame_executable_num_inputs": (c_int32, [c_void_p]),
    "frame_executable_num_outputs": (c_int32, [c_void_p]),
    "frame_executable_io_spec": (c_int32, [c_void_p, c_int32, c_int32, POINTER(c_int32), POINTER(c_int64),
                                           POINTER(c_int32)]),
    "frame_executable_run": (c_int32, [c_void_p, POINTER(c_void_p), c_int32, POINTER(c_void_p), c_int32, c_void_p]),
    "frame_executable_run_repeat": (c_int32, [c_void_p, POINTER(c_void_p), c_int32, c_int32, POINTER(c_void_p), c_int32,
                                              c_void_p, c_int32]),
    "frame_run_with_allocated_outputs": (c_int32, [c_void_p, POINTER(c_void_p), c_int32, POINTER(c_void_p), c_int32]),
    "frame_compile_cache_size": (c_int64, []),
    "frame_transform_text": (c_int32, [c_char_p, c_char_p, c_void_p, c_int64, POINTER(c_int64)]),
    "frame_roundtrip_text": (c_int32, [c_char_p, c_void_p, c_int64, POINTER(c_int64)]),
    "frame_memory_plan_text": (c_int32, [c_char_p, c_void_p, c_int64, POINTER(c_int64)]),
    "frame_hip_lowered_text": (c_int32, [c_char_p, c_int32, c_void_p, c_int64, POINTER(c_int64)]),
    "frame_backward_text": (c_int32, [c_char_p, c_int32, c_void_p, c_int32, c_void_p, c_int64, POINTER(c_int64)]),
    "frame_sgd_update_text": (c_int32, [c_char_p, c_void_p, c_int32, ctypes.c_double, c_void_p, c_int64, POINTER(c_int64)]),
    "frame_launch": (c_int32, [c_char_p, c_char_p, POINTER(c_void_p), c_int32, POINTER(c_void_p), c_int32, c_void_p]),
    "frame_backend_compile": (c_int32, [c_char_p, c_char_p, c_int32, POINTER(c_void_p)]),
    "frame_backend_copy": (c_int32, [c_char_p, c_void_p, c_char_p, c_int32, c_void_p, c_char_p, c_int32, c_size_t,
                                     c_void_p]),
    "frame_hip_allocator_stats": (c_int32, [c_int32, POINTER(ctypes.c_uint64)]),
    "frame_save_onnx_weights": (c_int32, [c_char_p, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "frame_load_onnx_weights": (c_int32, [c_char_p, POINTER(c_void_p)]),
    "frame_onnx_count": (c_int32, [c_void_p]),
    "frame_onnx_name": (c_char_p, [c_void_p, c_int32]),
    "frame_onnx_dtype": (c_int32, [c_void_p, c_int32]),
    "frame_onnx_rank": (c_int32, [c_void_p, c_int32]),
    "frame_onnx_dim": (c_int64, [c_void_p, c_int32, c_int32]),
    "frame_onnx_data": (c_void_p, [c_void_p, c_int32]),
    "frame_onnx_free": (None, [c_void_p]),
}


def lib() -> ctypes.CDLL:
    """Loads lib/libframe.so (global symbols, so plugins loaded later register into the same registries)."""
    global _lib
    if _lib is None:
        if not os.path.exists(HOST_LIB):
            raise FileNotFoundError(f"{HOST_LIB} is missing: run __graft_entry__.build() first")
        handle = ctypes.CDLL(HOST_LIB, mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGS.keys())


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = lib().frame_last_error().decode("utf-8", "replace")
        raise FrameError(rc, f"{what}: {msg}" if what else msg)


def _text(fn, *args) -> str:
    needed = c_int64(0)
    rc = fn(*args, None, 0, ctypes.byref(needed))
    if rc not in (0, -1):
        check(rc)
    buf = ctypes.create_string_buffer(needed.value)
    check(fn(*args, buf, needed.value, ctypes.byref(needed)))
    return buf.value.decode()


def backends() -> list[str]:
    s = _text(lib().frame_backends)
    return s.split(",") if s else []


def device_count(backend: str = "hip") -> int:
    n = c_int32(0)
    check(lib().frame_device_count(backend.encode(), ctypes.byref(n)), "frame_device_count")
    return n.value


def transform(ir_text: str, pass_name: str = "") -> str:
    return _text(lib().frame_transform_text, ir_text.encode(), pass_name.encode())


def hip_lowered(ir_text: str, opt_level: int = 1) -> str:
    """The graph the hip backend plans: standard pipeline, then HipBackend::compile's lowering (host only)."""
    return _text(lib().frame_hip_lowered_text, ir_text.encode(), opt_level)


def backward(ir_text: str, loss_index: int, wrt) -> str:
    """compiler::build_backward_graph on IR text: forward outputs, then d(output loss_index)/d(inputs wrt)."""
    idx = (ctypes.c_int32 * max(1, len(wrt)))(*wrt)
    return _text(lib().frame_backward_text, ir_text.encode(), loss_index, idx, len(wrt))


def sgd_update(ir_text: str, param_inputs, learning_rate: float) -> str:
    """compiler::build_sgd_update_graph for the types of graph inputs `param_inputs` of `ir_text`."""
    idx = (ctypes.c_int32 * max(1, len(param_inputs)))(*param_inputs)
    return _text(lib().frame_sgd_update_text, ir_text.encode(), idx, len(param_inputs), learning_rate)


def roundtrip(ir_text: str) -> str:
    return _text(lib().frame_roundtrip_text, ir_text.encode())


def memory_plan(ir_text: str) -> str:
    return _text(lib().frame_memory_plan_text, ir_text.encode())


def compile_cache_size() -> int:
    return lib().frame_compile_cache_size()


class Tensor:
    """A frame::Tensor allocated by a backend's allocator (device memory for hip)."""

    def __init__(self, backend: str, dtype: int, shape, device: int = 0, _handle=None, byte_offset: int = 0):
        """byte_offset > 0: a view that starts that many bytes into its own block (Tensor::from_storage_slice)."""
        self.backend, self.dtype, self.shape = backend, int(dtype), tuple(int(d) for d in shape)
        if _handle is None:
            h = c_void_p()
            dims = (c_int64 * max(1, len(self.shape)))(*self.shape)
            if byte_offset:
                check(lib().frame_tensor_empty_at(backend.encode(), device, self.dtype, dims, len(self.shape),
                                                  byte_offset, ctypes.byref(h)), "frame_tensor_empty_at")
            else:
                check(lib().frame_tensor_empty(backend.encode(), device, self.dtype, dims, len(self.shape),
                                               ctypes.byref(h)), "frame_tensor_empty")
            _handle = h
        self.handle = _handle

    @classmethod
    def from_numpy(cls, backend: str, dtype: int, array: np.ndarray, byte_offset: int = 0) -> "Tensor":
        a = np.ascontiguousarray(array, dtype=_NP[dtype])  # (ndim >= 1: a rank-0 array comes back as [1])
        t = cls(backend, dtype, np.shape(array), byte_offset=byte_offset)
        check(lib().frame_tensor_upload(t.handle, a.ctypes.data, a.nbytes), "frame_tensor_upload")
        return t

    @property
    def data_ptr(self) -> int:
        return lib().frame_tensor_data(self.handle) or 0

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=_NP[self.dtype])
        check(lib().frame_tensor_download(self.handle, out.ctypes.data, out.nbytes), "frame_tensor_download")
        return out

    def __del__(self):
        try:
            if _lib is not None and self.handle:
                _lib.frame_tensor_free(self.handle)
                self.handle = None
        except Exception:
            pass


class Stream:
    def __init__(self, backend: str = "hip", device: int = 0):
        self.handle = c_void_p()
        check(lib().frame_stream_create(backend.encode(), device, ctypes.byref(self.handle)), "frame_stream_create")

    @property
    def native(self) -> int:
        return lib().frame_stream_native(self.handle) or 0

    def synchronize(self) -> None:
        check(lib().frame_stream_synchronize(self.handle), "frame_stream_synchronize")

    def __del__(self):
        try:
            if _lib is not None and self.handle:
                _lib.frame_stream_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


def _ptrs(tensors):
    return (c_void_p * max(1, len(tensors)))(*[t.handle.value if isinstance(t.handle, c_void_p) else t.handle
                                               for t in tensors])


class Executable:
    """runtime::compile result; run() = runtime::run_with_allocated_outputs on numpy inputs."""

    def __init__(self, ir_text: str, backend: str, opt_level: int = 1):
        self.backend = backend
        self.handle = c_void_p()
        check(lib().frame_compile(ir_text.encode(), backend.encode(), opt_level, ctypes.byref(self.handle)),
              f"compile for {backend}")

    def _spec(self, is_output: int, i: int):
        dt, rank = c_int32(0), c_int32(0)
        dims = (c_int64 * 8)()
        check(lib().frame_executable_io_spec(self.handle, is_output, i, ctypes.byref(dt), dims, ctypes.byref(rank)))
        return dt.value, tuple(dims[k] for k in range(rank.value))

    def input_specs(self):
        return [self._spec(0, i) for i in range(lib().frame_executable_num_inputs(self.handle))]

    def output_specs(self):
        return [self._spec(1, i) for i in range(lib().frame_executable_num_outputs(self.handle))]

    def upload_inputs(self, arrays):
        specs = self.input_specs()
        assert len(arrays) == len(specs), (len(arrays), len(specs))
        return [a if isinstance(a, Tensor) else Tensor.from_numpy(self.backend, dt, a) for a, (dt, _) in zip(arrays, specs)]

    def alloc_outputs(self):
        return [Tensor(self.backend, dt, shape) for dt, shape in self.output_specs()]

    def run_tensors(self, inputs, outputs, stream: Stream) -> None:
        check(lib().frame_executable_run(self.handle, _ptrs(inputs), len(inputs), _ptrs(outputs), len(outputs),
                                         stream.handle), "Executable.run")

    def run_repeat(self, input_sets, outputs, stream: Stream, iterations: int) -> None:
        """frame_executable_run_repeat: `iterations` runs issued from native code, run i reading input_sets[i % n]."""
        flat = [t for s in input_sets for t in s]
        n_in = len(input_sets[0]) if input_sets else 0
        check(lib().frame_executable_run_repeat(self.handle, _ptrs(flat), len(input_sets), n_in, _ptrs(outputs),
                                                len(outputs), stream.handle, iterations), "Executable.run_repeat")

    def steps(self) -> list[str]:
        """The hip executable's plan steps: the op of each non-input node of the lowered graph, in order."""
        return [line.split(" ", 1)[1] for line in _text(lib().frame_hip_executable_steps, self.handle).splitlines()]

    def run_tapped(self, inputs, outputs, stream: Stream, taps) -> None:
        """frame_hip_run_tapped: taps = [(step, output index, numpy array sized like that output)]; each array is
        filled with the step's output as it was produced."""
        n = len(taps)
        steps = (c_int32 * max(1, n))(*[t[0] for t in taps])
        outs = (c_int32 * max(1, n))(*[t[1] for t in taps])
        hosts = (c_void_p * max(1, n))(*[t[2].ctypes.data for t in taps])
        sizes = (c_int64 * max(1, n))(*[t[2].nbytes for t in taps])
        check(lib().frame_hip_run_tapped(self.handle, _ptrs(inputs), len(inputs), _ptrs(outputs), len(outputs),
                                         stream.handle, n, steps, outs, hosts, sizes), "frame_hip_run_tapped")

    def run(self, inputs):
        """Inputs as numpy arrays (storage form) or Tensors; returns numpy outputs."""
        ins = self.upload_inputs(inputs)
        n_out = lib().frame_executable_num_outputs(self.handle)
        outs = (c_void_p * max(1, n_out))()
        check(lib().frame_run_with_allocated_outputs(self.handle, _ptrs(ins), len(ins), outs, n_out),
              "run_with_allocated_outputs")
        results = []
        for i, (dt, shape) in enumerate(self.output_specs()):
            t = Tensor(self.backend, dt, shape, _handle=c_void_p(outs[i]))
            results.append(t.numpy())
        return results

    def __del__(self):
        try:
            if _lib is not None and self.handle:
                _lib.frame_executable_free(self.handle)
                self.handle = None
        except Exception:
            pass


def backend_compile(graph, backend: str, opt_level: int = 1) -> Executable:
    """Backend::compile of the graph as given (no pass pipeline, no compile cache)."""
    text = graph if isinstance(graph, str) else graph.text()
    exe = Executable.__new__(Executable)
    exe.backend = backend
    exe.handle = c_void_p()
    check(lib().frame_backend_compile(text.encode(), backend.encode(), opt_level, ctypes.byref(exe.handle)),
          f"Backend::compile for {backend}")
    return exe


def backend_copy(backend: str, dst: int, dst_backend: str, src: int, src_backend: str, nbytes: int,
                 stream: "Stream | None" = None) -> None:
    """Backend::copy between raw addresses; "cpu" names host memory."""
    check(lib().frame_backend_copy(backend.encode(), c_void_p(dst), dst_backend.encode(), 0, c_void_p(src),
                                   src_backend.encode(), 0, nbytes, stream.handle if stream else None),
          "Backend::copy")


def allocator_stats(device: int = 0) -> dict:
    """The hip caching allocator's counters (bytes live / reusable / freed with work possibly queued, allocations,
    device-wide waits, waits on one freed block's fence)."""
    out = (ctypes.c_uint64 * 6)()
    check(lib().frame_hip_allocator_stats(device, out), "frame_hip_allocator_stats")
    return dict(zip(("live", "cached", "pending", "device_allocations", "device_syncs", "fence_waits"),
                    [int(v) for v in out]))


def onnx_arrays(weights):
    """(names, dtypes, dims, ranks, data) ctypes arrays for {name: (dtype, numpy array)} (kept alive by the caller)."""
    names = list(weights)
    # (np.ascontiguousarray would turn a rank-0 array into rank 1)
    arrs = [np.asarray(weights[n][1]).copy(order="C") for n in names]
    dims = [(c_int64 * max(1, a.ndim))(*a.shape) for a in arrs]
    c_names = (c_char_p * max(1, len(names)))(*[n.encode() for n in names])
    c_dtypes = (c_int32 * max(1, len(names)))(*[int(weights[n][0]) for n in names])
    c_dims = (c_void_p * max(1, len(names)))(*[ctypes.addressof(d) for d in dims])
    c_ranks = (c_int32 * max(1, len(names)))(*[a.ndim for a in arrs])
    c_data = (c_void_p * max(1, len(names)))(*[a.ctypes.data for a in arrs])
    return (c_names, c_dtypes, c_dims, c_ranks, c_data), (arrs, dims)


def save_onnx_weights(path: str, weights) -> None:
    """interop::save_onnx_weights: weights = {name: (dtype code, numpy array of its storage)}, in order."""
    args, keep = onnx_arrays(weights)
    check(lib().frame_save_onnx_weights(path.encode(), len(weights), *args), "save_onnx_weights")


def load_onnx_weights(path: str) -> dict:
    """interop::load_onnx_weights: {name: (dtype code, numpy array)} in file order."""
    h = c_void_p()
    check(lib().frame_load_onnx_weights(path.encode(), ctypes.byref(h)), "load_onnx_weights")
    try:
        out = {}
        for i in range(lib().frame_onnx_count(h)):
            dt = lib().frame_onnx_dtype(h, i)
            shape = tuple(lib().frame_onnx_dim(h, i, k) for k in range(lib().frame_onnx_rank(h, i)))
            a = np.empty(shape, dtype=_NP[dt])
            if a.nbytes:
                ctypes.memmove(a.ctypes.data, lib().frame_onnx_data(h, i), a.nbytes)
            out[lib().frame_onnx_name(h, i).decode()] = (dt, a)
        return out
    finally:
        lib().frame_onnx_free(h)


def compile(graph, backend: str, opt_level: int = 1) -> Executable:
    text = graph if isinstance(graph, str) else graph.text()
    return Executable(text, backend, opt_level)


def launch(node_ir_text: str, backend: str, inputs, outputs, stream: Stream | None = None) -> None:
    check(lib().frame_launch(node_ir_text.encode(), backend.encode(), _ptrs(inputs), len(inputs), _ptrs(outputs),
                             len(outputs), stream.handle if stream else None), "Backend.launch")

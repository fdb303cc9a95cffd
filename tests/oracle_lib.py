"""ctypes binding of the parity oracle (oracle/lib/liboracle_kernels.so) and of the reference build
(oracle/_ref/libframe_ref.so). Test infrastructure only."""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int8, c_int64, c_uint8, c_uint16, c_uint32, c_void_p

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_LIB = os.path.join(REPO, "oracle", "lib", "liboracle_kernels.so")
ORACLE_CPU_BACKEND = os.path.join(REPO, "oracle", "lib", "liboracle_cpu.so")
REF_LIB = os.path.join(REPO, "oracle", "_ref", "libframe_ref.so")

_oracle = None
_ref = None


def oracle() -> ctypes.CDLL:
    global _oracle
    if _oracle is None:
        lib = ctypes.CDLL(ORACLE_LIB)
        sigs = {
            "oracle_float_to_bf16": (c_uint16, [c_float]),
            "oracle_float_to_f16": (c_uint16, [c_float]),
            "oracle_bf16_to_float": (c_float, [c_uint16]),
            "oracle_f16_to_float": (c_float, [c_uint16]),
            "oracle_f32_to_bf16_array": (None, [c_void_p, c_void_p, c_int64]),
            "oracle_f32_to_f16_array": (None, [c_void_p, c_void_p, c_int64]),
            "oracle_matmul": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64]),
            "oracle_matmul_sample": (c_int, [c_int, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p,
                                             c_void_p, c_int64, c_void_p]),
            "oracle_conv2d": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
            "oracle_conv2d_sample": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
                                             c_void_p]),
            "oracle_ew_program": (c_int, [c_int, c_int, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int64]),
            "oracle_softmax": (c_int, [c_int, c_void_p, c_void_p, c_int64, c_int64]),
            "oracle_layer_norm": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64,
                                          c_double]),
            "oracle_pool2d": (c_int, [c_int, c_int, c_void_p, c_void_p, c_void_p]),
            "oracle_transpose": (c_int, [c_int, c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
            "oracle_slice": (c_int, [c_int, c_void_p, c_void_p, c_int, c_void_p, c_int64, c_int64, c_int64]),
            "oracle_concat": (c_int, [c_int, c_void_p, c_int, c_void_p, c_int, c_void_p, c_int64]),
            "oracle_constant": (c_int, [c_int, c_void_p, c_int64, c_void_p, c_int64]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _oracle = lib
    return _oracle


_cpu_backend = None


def load_cpu_backend() -> None:
    """Registers the oracle as Frame's `cpu` backend inside the already-loaded libframe.so."""
    global _cpu_backend
    if _cpu_backend is None:
        from frame_hip import host

        host.lib()
        _cpu_backend = ctypes.CDLL(ORACLE_CPU_BACKEND, mode=ctypes.RTLD_GLOBAL)


def run_graph_cpu(graph, inputs, opt_level: int = 1):
    """Compiles `graph` (a graphs.Graph on device 'cpu', or IR text) through runtime::compile for the oracle's
    cpu backend and runs it on host arrays."""
    from frame_hip import host

    load_cpu_backend()
    return host.compile(graph, "cpu", opt_level).run(inputs)


def ref_available() -> bool:
    return os.path.exists(REF_LIB)


def ref() -> ctypes.CDLL:
    global _ref
    if _ref is None:
        lib = ctypes.CDLL(REF_LIB, mode=ctypes.RTLD_LOCAL)
        sigs = {
            "ref_last_error": (c_char_p, []),
            "ref_float_to_bf16": (c_uint16, [c_float]),
            "ref_float_to_f16": (c_uint16, [c_float]),
            "ref_bf16_to_float": (c_float, [c_uint16]),
            "ref_f16_to_float": (c_float, [c_uint16]),
            "ref_compare_narrowing_exhaustive": (c_int64, [c_void_p, c_void_p, POINTER(c_uint32)]),
            "ref_run_graph": (c_int, [c_char_p, c_int, c_void_p, c_int, c_void_p]),
            "ref_transform_text": (c_int, [c_char_p, c_char_p, c_void_p, c_int64, POINTER(c_int64)]),
            "ref_roundtrip_text": (c_int, [c_char_p, c_void_p, c_int64, POINTER(c_int64)]),
            "ref_memory_plan_text": (c_int, [c_char_p, c_void_p, c_int64, POINTER(c_int64)]),
            "ref_backward_text": (c_int, [c_char_p, ctypes.c_int32, c_void_p, ctypes.c_int32, c_void_p, c_int64,
                                          POINTER(c_int64)]),
            "ref_sgd_update_text": (c_int, [c_char_p, c_void_p, ctypes.c_int32, ctypes.c_double, c_void_p, c_int64,
                                            POINTER(c_int64)]),
            "ref_save_onnx_weights": (c_int, [c_char_p, ctypes.c_int32, c_void_p, c_void_p, c_void_p, c_void_p,
                                              c_void_p]),
            "ref_load_onnx_weights": (c_int, [c_char_p]),
            "ref_onnx_count": (ctypes.c_int32, []),
            "ref_onnx_name": (c_char_p, [ctypes.c_int32]),
            "ref_onnx_dtype": (ctypes.c_int32, [ctypes.c_int32]),
            "ref_onnx_rank": (ctypes.c_int32, [ctypes.c_int32]),
            "ref_onnx_dim": (c_int64, [ctypes.c_int32, ctypes.c_int32]),
            "ref_onnx_data": (c_void_p, [ctypes.c_int32]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _ref = lib
    return _ref


def _ptrs(arrays):
    return (c_void_p * len(arrays))(*[a.ctypes.data for a in arrays])


def ref_error() -> str:
    return ref().ref_last_error().decode()


def ref_run_graph(ir_text: str, inputs, out_specs):
    """Runs IR text on the reference CPU backend. out_specs: list of (shape, numpy dtype)."""
    ins = [np.ascontiguousarray(a) for a in inputs]
    outs = [np.empty(shape, dtype=dt) for shape, dt in out_specs]
    rc = ref().ref_run_graph(ir_text.encode(), len(ins), _ptrs(ins), len(outs), _ptrs(outs))
    if rc != 0:
        raise RuntimeError(f"reference run failed ({rc}): {ref_error()}")
    return outs


def _text_call(fn, *args) -> str:
    needed = c_int64(0)
    rc = fn(*args, None, 0, ctypes.byref(needed))
    if rc not in (0, -1):
        raise RuntimeError(f"reference call failed ({rc}): {ref_error()}")
    buf = ctypes.create_string_buffer(needed.value)
    rc = fn(*args, buf, needed.value, ctypes.byref(needed))
    if rc != 0:
        raise RuntimeError(f"reference call failed ({rc}): {ref_error()}")
    return buf.value.decode()


def ref_transform(ir_text: str, pass_name: str = "") -> str:
    return _text_call(ref().ref_transform_text, ir_text.encode(), pass_name.encode())


def ref_backward(ir_text: str, loss_index: int, wrt) -> str:
    """The reference's build_backward_graph on IR text."""
    idx = (ctypes.c_int32 * max(1, len(wrt)))(*wrt)
    return _text_call(ref().ref_backward_text, ir_text.encode(), loss_index, idx, len(wrt))


def ref_sgd_update(ir_text: str, param_inputs, learning_rate: float) -> str:
    """The reference's build_sgd_update_graph for the types of the given graph inputs of `ir_text`."""
    idx = (ctypes.c_int32 * max(1, len(param_inputs)))(*param_inputs)
    return _text_call(ref().ref_sgd_update_text, ir_text.encode(), idx, len(param_inputs), learning_rate)


def ref_roundtrip(ir_text: str) -> str:
    return _text_call(ref().ref_roundtrip_text, ir_text.encode())


def ref_memory_plan(ir_text: str) -> str:
    return _text_call(ref().ref_memory_plan_text, ir_text.encode())


# ---- convenience wrappers over the oracle -------------------------------------------------------------------

def storage_np(dtype: int):
    return np.float32 if dtype == 0 else np.uint16


def matmul(dtype, a, b):
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), dtype=storage_np(dtype))
    assert oracle().oracle_matmul(dtype, a.ctypes.data, b.ctypes.data, c.ctypes.data, m, n, k) == 0
    return c


def matmul_sample(dtype, a, b, rows, cols):
    m, k = a.shape
    n = b.shape[1]
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    cols = np.ascontiguousarray(cols, dtype=np.int64)
    out = np.empty(len(rows), dtype=storage_np(dtype))
    assert oracle().oracle_matmul_sample(dtype, a.ctypes.data, b.ctypes.data, m, n, k, rows.ctypes.data,
                                         cols.ctypes.data, len(rows), out.ctypes.data) == 0
    return out


def conv_out_hw(geom):
    n, cin, h, w, cout, kh, kw, sh, sw, ph, pw, g = geom
    return (h + 2 * ph - kh) // sh + 1, (w + 2 * pw - kw) // sw + 1


def conv2d(dtype, x, w, bias, geom):
    oh, ow = conv_out_hw(geom)
    y = np.empty((geom[0], geom[4], oh, ow), dtype=storage_np(dtype))
    g = np.asarray(geom, dtype=np.int64)
    assert oracle().oracle_conv2d(dtype, x.ctypes.data, w.ctypes.data, None if bias is None else bias.ctypes.data,
                                  y.ctypes.data, g.ctypes.data) == 0
    return y


def conv2d_sample(dtype, x, w, bias, geom, idx):
    g = np.asarray(geom, dtype=np.int64)
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    out = np.empty(len(idx), dtype=storage_np(dtype))
    assert oracle().oracle_conv2d_sample(dtype, x.ctypes.data, w.ctypes.data,
                                         None if bias is None else bias.ctypes.data, g.ctypes.data,
                                         idx.ctypes.data, len(idx), out.ctypes.data) == 0
    return out


def ew_program(dtype, ops, arities, ins):
    ins = [np.ascontiguousarray(a) for a in ins]
    out = np.empty_like(ins[0])
    o = (c_uint8 * len(ops))(*ops)
    ar = (c_int8 * len(arities))(*arities)
    assert oracle().oracle_ew_program(dtype, len(ops), o, ar, _ptrs(ins), len(ins), out.ctypes.data,
                                      ins[0].size) == 0
    return out


def softmax(dtype, x):
    y = np.empty_like(x)
    assert oracle().oracle_softmax(dtype, x.ctypes.data, y.ctypes.data, x.shape[0], x.shape[1]) == 0
    return y


def layer_norm(dtype, x, g, b, eps):
    y = np.empty_like(x)
    assert oracle().oracle_layer_norm(dtype, x.ctypes.data, g.ctypes.data, b.ctypes.data, y.ctypes.data,
                                      x.shape[0], x.shape[1], eps) == 0
    return y


def pool2d(dtype, mode, x, geom):
    n, c, h, w, kh, kw, sh, sw, ph, pw = geom
    oh, ow = (h + 2 * ph - kh) // sh + 1, (w + 2 * pw - kw) // sw + 1
    y = np.empty((n, c, oh, ow), dtype=x.dtype)
    g = np.asarray(geom, dtype=np.int64)
    rc = oracle().oracle_pool2d(dtype, mode, x.ctypes.data, y.ctypes.data, g.ctypes.data)
    if rc != 0:
        raise ValueError(f"oracle_pool2d rc={rc}")
    return y


def ref_save_onnx_weights(path: str, weights) -> None:
    """The reference's interop::save_onnx_weights on {name: (dtype code, numpy array)}."""
    from frame_hip import host

    args, keep = host.onnx_arrays(weights)
    if ref().ref_save_onnx_weights(path.encode(), len(weights), *args) != 0:
        raise RuntimeError(f"reference save_onnx_weights failed: {ref_error()}")


def ref_load_onnx_weights(path: str) -> dict:
    """The reference's interop::load_onnx_weights: {name: (dtype code, numpy array)} in file order."""
    r = ref()
    if r.ref_load_onnx_weights(path.encode()) != 0:
        raise RuntimeError(f"reference load_onnx_weights failed: {ref_error()}")
    out = {}
    for i in range(r.ref_onnx_count()):
        dt = r.ref_onnx_dtype(i)
        shape = tuple(r.ref_onnx_dim(i, k) for k in range(r.ref_onnx_rank(i)))
        a = np.empty(shape, dtype=storage_np(dt))
        if a.nbytes:
            ctypes.memmove(a.ctypes.data, r.ref_onnx_data(i), a.nbytes)
        out[r.ref_onnx_name(i).decode()] = (dt, a)
    return out

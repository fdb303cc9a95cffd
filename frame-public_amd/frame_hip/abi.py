"""ctypes binding of the gfx950 kernel library's C ABI (include/frame_hip_abi.h).

This is the plumbing the tests and the benchmark use to move host data into HBM and to call the kernels
directly. It loads only the in-tree library (frame-public_amd/lib/libframe_hip_kernels.so) and raises if it
is missing: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int8, c_int32, c_int64, c_size_t, c_uint8, c_uint64, c_void_p

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(PKG_DIR, "lib")
KERNELS_LIB = os.path.join(LIB_DIR, "libframe_hip_kernels.so")

FH_OK = 0
F32, F16, BF16 = 0, 2, 3
EW_ADD, EW_MUL, EW_RELU, EW_SQUARE, EW_GELU = 1, 2, 3, 4, 5
GEMM_ANY_ORDER = 1
H2H, H2D, D2H, D2D = 0, 1, 2, 3
MAX_SEGMENTS = 8

STATUS_NAMES = {0: "ok", 1: "invalid_argument", 2: "not_found", 4: "unimplemented", 5: "out_of_memory",
                6: "internal", 7: "device_error"}


class FrameHipError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{STATUS_NAMES.get(code, code)}] {message}")
        self.code = code


class Epilogue(ctypes.Structure):
    _fields_ = [("nseg", c_int32), ("round_between", c_int32), ("ops", c_uint8 * MAX_SEGMENTS),
                ("ins", c_void_p * MAX_SEGMENTS)]


_lib = None

# name -> (restype, argtypes)
_SIGS = {
    "fh_last_error": (c_char_p, []),
    "fh_abi_version": (c_int32, []),
    "fh_device_count": (c_int32, [POINTER(c_int32)]),
    "fh_set_device": (c_int32, [c_int32]),
    "fh_malloc": (c_int32, [POINTER(c_void_p), c_size_t, c_int32]),
    "fh_free": (c_int32, [c_void_p]),
    "fh_host_alloc": (c_int32, [POINTER(c_void_p), c_size_t]),
    "fh_host_free": (c_int32, [c_void_p]),
    "fh_memcpy": (c_int32, [c_void_p, c_void_p, c_size_t, c_int32, c_void_p]),
    "fh_stream_create": (c_int32, [POINTER(c_void_p), c_int32]),
    "fh_stream_destroy": (c_int32, [c_void_p]),
    "fh_stream_synchronize": (c_int32, [c_void_p]),
    "fh_device_synchronize": (c_int32, []),
    "fh_event_create": (c_int32, [POINTER(c_void_p), c_int32]),
    "fh_event_destroy": (c_int32, [c_void_p]),
    "fh_event_record": (c_int32, [c_void_p, c_void_p]),
    "fh_stream_wait_event": (c_int32, [c_void_p, c_void_p]),
    "fh_event_query": (c_int32, [c_void_p, POINTER(c_int32)]),
    "fh_event_synchronize": (c_int32, [c_void_p]),
    "fh_event_elapsed_ms": (c_int32, [c_void_p, c_void_p, POINTER(c_float)]),
    "fh_gemm": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, POINTER(Epilogue),
                          c_void_p]),
    "fh_conv2d_nchw_in_supported": (c_int32, [c_int32, POINTER(c_int64)]),
    "fh_conv2d_w_oihw_supported": (c_int32, [c_int32, POINTER(c_int64), POINTER(Epilogue)]),
    "fh_gemm_ex": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, POINTER(Epilogue),
                             c_int32, c_void_p]),
    "fh_gemm_grouped": (c_int32, [c_int32, c_void_p, c_int32, POINTER(c_void_p), POINTER(c_void_p), c_int64, c_int64,
                                  c_int64, POINTER(Epilogue), c_int32, c_void_p]),
    "fh_gemm_batched": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64,
                                  c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p]),
    "fh_conv2d_fwd": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_void_p, POINTER(c_int64),
                                POINTER(Epilogue), c_void_p]),
    "fh_conv2d_nhwc_fwd": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_void_p, POINTER(c_int64),
                                     POINTER(Epilogue), c_void_p]),
    "fh_conv2d_nhwc_supported": (c_int32, [c_int32, POINTER(c_int64)]),
    "fh_transpose_batched": (c_int32, [c_int32, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p]),
    "fh_conv_pack_input_c8": (c_int32, [c_void_p, c_void_p, c_int64, c_int32, c_int64, c_void_p]),
    "fh_conv_pack_filter_c8": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p]),
    "fh_conv2d_stem_pool_supported": (c_int32, [c_int32, POINTER(c_int64), POINTER(c_int64)]),
    "fh_conv2d_stem_pool": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_void_p, POINTER(c_int64),
                                      POINTER(c_int64), c_int32, c_void_p]),
    "fh_stream_capturing": (c_int32, [c_void_p, POINTER(c_int32)]),
    "fh_conv_c8_filter_k": (c_int64, [c_int64, c_int64]),
    "fh_transpose_planes_multi": (c_int32, [c_int32, c_int32, POINTER(c_void_p), POINTER(c_void_p), POINTER(c_int64),
                                            POINTER(c_int64), POINTER(c_int64), c_void_p]),
    "fh_ew_program": (c_int32, [c_int32, c_int32, POINTER(c_uint8), POINTER(c_int8), POINTER(c_void_p), c_int32,
                                c_void_p, c_int64, c_int32, c_void_p]),
    "fh_attention_fwd": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64,
                                   c_float, c_void_p]),
    "fh_attention_supported": (c_int32, [c_int32, c_int64, c_int64]),
    "fh_softmax_rows": (c_int32, [c_int32, c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "fh_layer_norm_rows": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_float,
                                     c_void_p]),
    "fh_graph_begin_capture": (c_int32, [c_void_p]),
    "fh_graph_end_capture": (c_int32, [c_void_p, c_int32, POINTER(c_void_p)]),
    "fh_graph_launch": (c_int32, [c_void_p, c_void_p]),
    "fh_graph_destroy": (c_int32, [c_void_p]),
    "fh_pool2d_nhwc": (c_int32, [c_int32, c_int32, c_void_p, c_void_p, POINTER(c_int64), c_void_p]),
    "fh_matmul_grad": (c_int32, [c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p]),
    "fh_pool2d_grad": (c_int32, [c_int32, c_int32, c_void_p, c_void_p, c_void_p, POINTER(c_int64), c_void_p]),
    "fh_conv2d_grad_input": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, POINTER(c_int64), c_void_p]),
    "fh_conv2d_grad_filter": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, POINTER(c_int64), c_void_p]),
    "fh_conv2d_wgrad_workspace": (c_int64, [c_int32, POINTER(c_int64), c_int32, POINTER(c_int32)]),
    "fh_conv2d_wgrad_nhwc_noalloc": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, POINTER(c_int64), c_int32,
                                               c_void_p]),
    "fh_conv2d_wgrad_nhwc": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, POINTER(c_int64), c_int32,
                                       c_void_p]),
    "fh_axpy_multi": (c_int32, [c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "fh_conv_filter_flip": (c_int32, [c_int32, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p]),
    "fh_conv_filter_flip_multi": (c_int32, [c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p]),
    "fh_dilate_nhwc": (c_int32, [c_int32, c_int32, c_void_p, c_void_p] + [c_int64] * 8 + [c_void_p]),
    "fh_avg_pool2d_grad_nhwc": (c_int32, [c_int32, c_void_p, c_void_p, POINTER(c_int64), c_void_p]),
    "fh_sum_rows_workspace": (c_int64, [c_int32, c_int64, c_int64]),
    "fh_sum_rows": (c_int32, [c_int32, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p]),
    "fh_sum": (c_int32, [c_int32, c_void_p, c_void_p, c_int32, POINTER(c_int64), c_void_p, c_void_p]),
    "fh_sum_grad": (c_int32, [c_int32, c_void_p, c_void_p, c_int32, POINTER(c_int64), c_void_p, c_void_p]),
    "fh_mse_loss": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_int64, c_void_p]),
    "fh_mse_loss_grad": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p]),
    "fh_conv2d_nhwc_fwd_ex": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_void_p, POINTER(c_int64), c_void_p,
                                        c_int32, c_void_p]),
    "fh_conv2d_nhwc_split_workspace": (c_int64, [c_int32, POINTER(c_int64), c_int32, POINTER(c_int32)]),
    "fh_conv2d_nhwc_fwd_split": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_void_p, POINTER(c_int64), c_void_p,
                                           c_int32, c_int32, c_void_p, c_int64, c_void_p]),
    "fh_pool2d": (c_int32, [c_int32, c_int32, c_void_p, c_void_p, POINTER(c_int64), c_void_p]),
    "fh_permute": (c_int32, [c_int32, c_void_p, c_void_p, c_int32, POINTER(c_int64), POINTER(c_int64), c_void_p]),
    "fh_copy2d": (c_int32, [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64, c_void_p]),
    "fh_fill": (c_int32, [c_void_p, c_int32, c_uint64, c_int64, c_void_p]),
}


def lib() -> ctypes.CDLL:
    """Loads the in-tree kernel library (raises when it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(KERNELS_LIB):
            raise FileNotFoundError(f"{KERNELS_LIB} is missing: run __graft_entry__.build() first")
        handle = ctypes.CDLL(KERNELS_LIB, mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGS.keys())


def check(code: int, what: str = "") -> None:
    if code != FH_OK:
        msg = lib().fh_last_error().decode("utf-8", "replace")
        raise FrameHipError(code, f"{what}: {msg}" if what else msg)


def device_count() -> int:
    n = c_int32(0)
    check(lib().fh_device_count(ctypes.byref(n)), "fh_device_count")
    return n.value


def storage_dtype(dtype: int):
    return np.float32 if dtype == F32 else np.uint16


class DeviceBuffer:
    """Owned device allocation (fh_malloc / fh_free)."""

    def __init__(self, nbytes: int, device: int = 0):
        self.nbytes = int(nbytes)
        self.ptr = c_void_p()
        check(lib().fh_malloc(ctypes.byref(self.ptr), max(self.nbytes, 1), device), "fh_malloc")

    @property
    def value(self) -> int:
        return self.ptr.value

    def upload(self, array: np.ndarray, stream=None) -> "DeviceBuffer":
        a = np.ascontiguousarray(array)
        assert a.nbytes <= self.nbytes, (a.nbytes, self.nbytes)
        check(lib().fh_memcpy(self.ptr, a.ctypes.data, a.nbytes, H2D, stream), "fh_memcpy H2D")
        return self

    def download(self, shape, dtype, stream=None) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        check(lib().fh_memcpy(out.ctypes.data, self.ptr, out.nbytes, D2H, stream), "fh_memcpy D2H")
        return out

    def free(self) -> None:
        if self.ptr.value:
            check(lib().fh_free(self.ptr), "fh_free")
            self.ptr = c_void_p()

    def __del__(self):
        try:
            if _lib is not None and self.ptr.value:
                _lib.fh_free(self.ptr)
        except Exception:
            pass


def to_device(array: np.ndarray) -> DeviceBuffer:
    a = np.ascontiguousarray(array)
    return DeviceBuffer(a.nbytes).upload(a)


class Stream:
    def __init__(self, device: int = 0):
        self.ptr = c_void_p()
        check(lib().fh_stream_create(ctypes.byref(self.ptr), device), "fh_stream_create")

    def synchronize(self) -> None:
        check(lib().fh_stream_synchronize(self.ptr), "fh_stream_synchronize")

    def __del__(self):
        try:
            if _lib is not None and self.ptr.value:
                _lib.fh_stream_destroy(self.ptr)
        except Exception:
            pass


class Event:
    def __init__(self, device: int = 0):
        self.ptr = c_void_p()
        check(lib().fh_event_create(ctypes.byref(self.ptr), device), "fh_event_create")

    def record(self, stream: Stream | None) -> None:
        check(lib().fh_event_record(self.ptr, stream.ptr if stream else None), "fh_event_record")

    def synchronize(self) -> None:
        check(lib().fh_event_synchronize(self.ptr), "fh_event_synchronize")

    def elapsed_ms(self, later: "Event") -> float:
        ms = c_float(0.0)
        check(lib().fh_event_elapsed_ms(self.ptr, later.ptr, ctypes.byref(ms)), "fh_event_elapsed_ms")
        return ms.value

    def __del__(self):
        try:
            if _lib is not None and self.ptr.value:
                _lib.fh_event_destroy(self.ptr)
        except Exception:
            pass


def make_epilogue(segments) -> Epilogue:
    """segments: list of (op_code, operand_device_ptr_or_None)."""
    ep = Epilogue()
    ep.nseg = len(segments)
    ep.round_between = 1
    for i, (op, ptr) in enumerate(segments):
        ep.ops[i] = op
        ep.ins[i] = ptr
    return ep


def i64_array(values):
    return (c_int64 * len(values))(*[int(v) for v in values])

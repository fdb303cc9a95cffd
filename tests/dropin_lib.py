"""ctypes binding of oracle/_ref/libframe_dropin.so: the reference's own runtime (runtime::compile with its cache,
the nine-pass pipeline, FallbackExecutable, run_with_allocated_outputs, the cpu backend) linked with this
repository's hip plugin sources compiled unchanged against the reference's headers (oracle/Makefile, target
dropin; oracle/dropin_driver.cpp). Test infrastructure only: the library is built in the container that holds
the reference and travels to the GPU box with the tree like oracle/_ref/libframe_ref.so."""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_int32, c_int64, c_void_p

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DROPIN_LIB = os.path.join(REPO, "oracle", "_ref", "libframe_dropin.so")
_NP = {0: np.float32, 2: np.uint16, 3: np.uint16}

_lib = None


def available() -> bool:
    return os.path.exists(DROPIN_LIB)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        d = ctypes.CDLL(DROPIN_LIB)
        sigs = {
            "dropin_last_error": (c_char_p, []),
            "dropin_backends": (c_int32, [c_char_p, c_int64]),
            "dropin_device_count": (c_int32, [c_char_p, POINTER(c_int32)]),
            "dropin_compile": (c_int32, [c_char_p, c_char_p, c_int32, POINTER(c_void_p)]),
            "dropin_free": (None, [c_void_p]),
            "dropin_identity": (c_void_p, [c_void_p]),
            "dropin_num_io": (c_int32, [c_void_p, c_int32]),
            "dropin_io_spec": (c_int32, [c_void_p, c_int32, c_int32, POINTER(c_int32), POINTER(c_int64),
                                         POINTER(c_int32)]),
            "dropin_run": (c_int32, [c_void_p, POINTER(c_void_p), c_int32, POINTER(c_void_p), c_int32]),
            "dropin_run_host_inputs": (c_int32, [c_void_p, POINTER(c_void_p), c_int32]),
            "dropin_fallback_count": (c_int64, [c_char_p, c_char_p]),
            "dropin_sandwich_op": (c_char_p, []),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(d, name)
            fn.restype = res
            fn.argtypes = args
        _lib = d
    return _lib


class DropinError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code, self.message = code, message


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise DropinError(rc, f"{what}: {lib().dropin_last_error().decode('utf-8', 'replace')}")


def backends() -> list[str]:
    buf = ctypes.create_string_buffer(256)
    check(lib().dropin_backends(buf, 256), "dropin_backends")
    return buf.value.decode().split(",")


def device_count(backend: str) -> int:
    n = c_int32(0)
    check(lib().dropin_device_count(backend.encode(), ctypes.byref(n)), "dropin_device_count")
    return n.value


def fallback_count(op: str, backend: str = "hip") -> int:
    return lib().dropin_fallback_count(op.encode(), backend.encode())


def sandwich_op() -> str:
    return lib().dropin_sandwich_op().decode()


class Executable:
    """runtime::compile(parse_text(text), backend, {opt_level}) of the reference runtime."""

    def __init__(self, text: str, backend: str, opt_level: int = 1):
        self.handle = c_void_p()
        check(lib().dropin_compile(text.encode(), backend.encode(), opt_level, ctypes.byref(self.handle)),
              f"runtime::compile for {backend}")

    def identity(self) -> int:
        return lib().dropin_identity(self.handle) or 0

    def specs(self, is_output: int):
        out = []
        for i in range(lib().dropin_num_io(self.handle, is_output)):
            dt, rank = c_int32(0), c_int32(0)
            dims = (c_int64 * 8)()
            check(lib().dropin_io_spec(self.handle, is_output, i, ctypes.byref(dt), dims, ctypes.byref(rank)), "spec")
            out.append((dt.value, tuple(dims[k] for k in range(rank.value))))
        return out

    def run(self, inputs):
        """runtime::run_with_allocated_outputs on device 0, inputs copied from and outputs back to numpy arrays."""
        ins = [np.ascontiguousarray(a) for a in inputs]
        outs = [np.empty(shape, _NP[dt]) for dt, shape in self.specs(1)]
        pin = (c_void_p * max(1, len(ins)))(*[a.ctypes.data for a in ins])
        pout = (c_void_p * max(1, len(outs)))(*[o.ctypes.data for o in outs])
        check(lib().dropin_run(self.handle, pin, len(ins), pout, len(outs)), "run_with_allocated_outputs")
        return outs

    def run_with_host_inputs(self, inputs) -> tuple[int, str]:
        """Executable::run with cpu tensors as inputs: (status code, message)."""
        ins = [np.ascontiguousarray(a) for a in inputs]
        pin = (c_void_p * max(1, len(ins)))(*[a.ctypes.data for a in ins])
        rc = lib().dropin_run_host_inputs(self.handle, pin, len(ins))
        return rc, lib().dropin_last_error().decode("utf-8", "replace")

    def __del__(self):
        try:
            if _lib is not None and self.handle:
                _lib.dropin_free(self.handle)
                self.handle = None
        except Exception:
            pass

"""frame_hip — Python plumbing of the MI355X `hip` backend plugin for Frame.

abi:     ctypes binding of the kernel library's C ABI (include/frame_hip_abi.h).
runtime: ctypes binding of the host runtime's C API (include/frame_capi.h): compile Frame IR text for a
         backend and run the resulting Executable on device buffers.
"""
from . import abi  # noqa: F401

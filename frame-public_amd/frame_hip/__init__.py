"""frame_hip — Python plumbing of the MI355X `hip` backend plugin for Frame.

abi:    ctypes binding of the kernel library's C ABI (include/frame_hip_abi.h), for direct kernel calls.
host:   ctypes binding of the host library's C API (include/frame_capi.h): compile Frame IR text for a backend
        through runtime::compile and run the Executable.
graphs: IR text builders for the benchmark configurations.
synth:  the seeded input generator shared by tests and the benchmark.
"""
from . import abi, graphs, host, synth  # noqa: F401

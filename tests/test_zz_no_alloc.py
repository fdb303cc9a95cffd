"""fh_conv2d_wgrad_nhwc_noalloc, the filter gradient that allocates nothing (its split-K partials live in a
file-scope device array), against fh_conv2d_wgrad_nhwc with a caller workspace, through the C ABI: two calls in a
row, the second on a smaller input, each bit-identical to the workspace entry point (same split count, same
summation order). Also: a geometry whose partials exceed the 64 MiB scratch is rejected on the host.
"""
import ctypes

import numpy as np
import pytest

from frame_hip import abi, synth
from tolerance import assert_bitwise

pytestmark = pytest.mark.gpu
BF16 = 3


def say(msg):
    print(f"[case] {msg}", flush=True)


def nhwc(a):
    return np.ascontiguousarray(np.transpose(a, (0, 2, 3, 1)))


def run_both(geom, seed):
    n, cin, h, w, cout, kh, kw, sh, sw, ph, pw, _ = geom
    oh, ow = (h + 2 * ph - kh) // sh + 1, (w + 2 * pw - kw) // sw + 1
    x = nhwc(synth.tensor(seed, (n, cin, h, w), BF16, "normal"))
    dy = nhwc(synth.tensor(seed + 1, (n, cout, oh, ow), BF16, "normal"))
    g = abi.i64_array(geom)
    lib = abi.lib()
    splits = ctypes.c_int32(0)
    need = lib.fh_conv2d_wgrad_workspace(BF16, g, cin, ctypes.byref(splits))
    assert need > 0
    dx, ddy = abi.to_device(x), abi.to_device(dy)
    dw_ref, dw_na = abi.DeviceBuffer(cout * cin * kh * kw * 2), abi.DeviceBuffer(cout * cin * kh * kw * 2)
    ws = abi.DeviceBuffer(need)
    s = abi.Stream()
    abi.check(lib.fh_conv2d_wgrad_nhwc(BF16, dx.ptr, ddy.ptr, dw_ref.ptr, ws.ptr, need, g, cin, s.ptr), "wgrad")
    abi.check(lib.fh_conv2d_wgrad_nhwc_noalloc(BF16, dx.ptr, ddy.ptr, dw_na.ptr, g, cin, s.ptr), "wgrad noalloc")
    s.synchronize()
    shape = (cout, cin, kh, kw)
    return dw_ref.download(shape, np.uint16), dw_na.download(shape, np.uint16), need, splits.value


def test_noalloc_wgrad_matches_workspace_entry_point_twice_second_smaller():
    for call, (geom, seed) in enumerate([((16, 64, 28, 28, 128, 3, 3, 1, 1, 1, 1, 1), 71),
                                         ((2, 32, 9, 11, 64, 3, 3, 2, 2, 1, 1, 1), 73)]):
        want, got, need, splits = run_both(geom, seed)
        say(f"call {call}: geometry {geom}, {splits} splits, {need} bytes of partials")
        assert_bitwise(got, want, f"no-alloc filter gradient, call {call}")


def test_noalloc_wgrad_rejects_partials_above_the_scratch():
    geom = (1, 2048, 8, 8, 2048, 3, 3, 1, 1, 1, 1, 1)
    lib = abi.lib()
    need = lib.fh_conv2d_wgrad_workspace(BF16, abi.i64_array(geom), 2048, None)
    assert need > (64 << 20), need
    tiny = abi.DeviceBuffer(256)
    rc = lib.fh_conv2d_wgrad_nhwc_noalloc(BF16, tiny.ptr, tiny.ptr, tiny.ptr, abi.i64_array(geom), 2048, None)
    assert rc == 1, rc  # FH_INVALID_ARGUMENT, before anything is launched
    assert b"no-allocation scratch" in lib.fh_last_error()


def test_noalloc_wgrad_calls_on_two_streams_are_ordered():
    """Two calls on two streams with no synchronisation between them share the device's scratch array: the second
    call's stream waits for the first call's kernels, so both gradients equal the workspace entry point's."""
    geom = (16, 64, 28, 28, 128, 3, 3, 1, 1, 1, 1, 1)
    n, cin, h, w, cout, kh, kw = geom[:7]
    lib = abi.lib()
    g = abi.i64_array(geom)
    need = lib.fh_conv2d_wgrad_workspace(BF16, g, cin, None)
    ws = abi.DeviceBuffer(need)
    cases = []
    for seed in (81, 83):
        x = abi.to_device(nhwc(synth.tensor(seed, (n, cin, h, w), BF16, "normal")))
        dy = abi.to_device(nhwc(synth.tensor(seed + 1, (n, cout, h, w), BF16, "normal")))
        cases.append((x, dy, abi.DeviceBuffer(cout * cin * kh * kw * 2), abi.DeviceBuffer(cout * cin * kh * kw * 2)))
    s_ref, s1, s2 = abi.Stream(), abi.Stream(), abi.Stream()
    for x, dy, ref, _ in cases:
        abi.check(lib.fh_conv2d_wgrad_nhwc(BF16, x.ptr, dy.ptr, ref.ptr, ws.ptr, need, g, cin, s_ref.ptr), "wgrad")
        s_ref.synchronize()
    say("two no-alloc calls on two streams, back to back")
    for (x, dy, _, out), s in zip(cases, (s1, s2)):
        abi.check(lib.fh_conv2d_wgrad_nhwc_noalloc(BF16, x.ptr, dy.ptr, out.ptr, g, cin, s.ptr), "wgrad noalloc")
    s1.synchronize()
    s2.synchronize()
    shape = (cout, cin, kh, kw)
    for i, (_, _, ref, out) in enumerate(cases):
        assert_bitwise(out.download(shape, np.uint16), ref.download(shape, np.uint16), f"stream {i + 1}")

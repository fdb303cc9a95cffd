"""ONNX weight exchange (interop::save_onnx_weights / load_onnx_weights; reference
include/frame/interop/onnx_weights.h:38,47, src/interop/onnx_weights.cpp, tests
tests/cpp/interop/test_onnx_weights.cpp:181-370), host-only.

Pins: files written here are byte-identical to the reference build's (oracle/_ref, compiled from the reference's
own src/interop/onnx_weights.cpp) for seeded float32 / float16 / bfloat16 tensors, and each side loads the other's
files bit for bit; the error cases of the reference's tests give the same error codes; unknown fields of every
supported wire type are skipped. Independent of the reference: a hand-assembled protobuf (the published ONNX
field numbers) decodes to the expected tensor.
"""
import os
import struct

import numpy as np
import pytest

import oracle_lib as orc
from frame_hip import host, synth

F32, F16, BF16, I32 = 0, 2, 3, 6


def weights(seed=7):
    return {
        "w1": (F32, synth.tensor(seed, (784, 256), F32, "normal")),
        "b1": (BF16, synth.tensor(seed + 1, (256,), BF16, "normal")),
        "h": (F16, synth.tensor(seed + 2, (3, 5, 7), F16, "normal")),
        "scalar": (F32, np.array(1.5, np.float32)),
        "empty": (BF16, np.zeros((0, 4), np.uint16)),
    }


def assert_same(got, want):
    assert list(got) == list(want), (list(got), list(want))
    for k in want:
        assert got[k][0] == want[k][0], k
        a, b = np.asarray(got[k][1]), np.asarray(want[k][1])
        assert a.shape == b.shape, (k, a.shape, b.shape)
        assert a.tobytes() == b.tobytes(), k


def test_round_trip_three_dtypes(tmp_path):
    p = str(tmp_path / "w.onnx")
    host.save_onnx_weights(p, weights())
    assert_same(host.load_onnx_weights(p), weights())


@pytest.mark.skipif(not orc.ref_available(), reason="oracle/_ref not built (no /root/reference here)")
def test_files_are_byte_identical_to_the_reference_and_cross_load(tmp_path):
    ours, theirs = str(tmp_path / "ours.onnx"), str(tmp_path / "ref.onnx")
    host.save_onnx_weights(ours, weights())
    orc.ref_save_onnx_weights(theirs, weights())
    assert open(ours, "rb").read() == open(theirs, "rb").read()
    assert_same(orc.ref_load_onnx_weights(ours), weights())
    assert_same(host.load_onnx_weights(theirs), weights())


def pb_varint(v):
    out = bytearray()
    while v >= 0x80:
        out.append((v & 0x7F) | 0x80)
        v >>= 7
    out.append(v)
    return bytes(out)


def pb_field(num, wire, payload):
    key = pb_varint((num << 3) | wire)
    if wire == 2:
        return key + pb_varint(len(payload)) + payload
    return key + payload


def test_hand_assembled_model_decodes():
    # TensorProto{dims=[2,3], data_type=FLOAT, name="t", raw_data=6 floats} in GraphProto.initializer (5) in
    # ModelProto.graph (7), plus unknown fields of wire types 0, 1, 2 and 5 at every level
    vals = np.arange(6, dtype=np.float32) * 0.25
    unknown = pb_field(99, 0, pb_varint(300)) + pb_field(98, 1, b"\0" * 8) + pb_field(97, 2, b"xyz") + \
        pb_field(96, 5, b"\1\2\3\4")
    tensor = pb_field(1, 0, pb_varint(2)) + pb_field(1, 0, pb_varint(3)) + pb_field(2, 0, pb_varint(1)) + unknown + \
        pb_field(8, 2, b"t") + pb_field(9, 2, vals.tobytes())
    graph = unknown + pb_field(2, 2, b"g") + pb_field(5, 2, tensor)
    model = pb_field(1, 0, pb_varint(8)) + unknown + pb_field(7, 2, graph)
    path = "/tmp/frame_onnx_hand.onnx"
    open(path, "wb").write(model)
    got = host.load_onnx_weights(path)
    assert list(got) == ["t"] and got["t"][0] == F32
    assert np.array_equal(got["t"][1], vals.reshape(2, 3))
    os.remove(path)


def expect_error(fn, code, *fragments):
    with pytest.raises(host.FrameError) as e:
        fn()
    msg = str(e.value)
    assert msg.startswith(f"[{code}]"), msg
    for f in fragments:
        assert f in msg, msg


def test_error_cases_match_the_reference_contract(tmp_path):
    expect_error(lambda: host.load_onnx_weights(str(tmp_path / "missing.onnx")), "not_found")
    good = str(tmp_path / "w.onnx")
    host.save_onnx_weights(good, weights())
    data = open(good, "rb").read()
    cut = str(tmp_path / "cut.onnx")
    open(cut, "wb").write(data[:len(data) // 2])
    expect_error(lambda: host.load_onnx_weights(cut), "invalid_argument")
    grp = str(tmp_path / "group.onnx")
    open(grp, "wb").write(pb_field(1, 0, pb_varint(8)) + pb_varint((5 << 3) | 3))
    expect_error(lambda: host.load_onnx_weights(grp), "unimplemented", "group")
    bad_type = str(tmp_path / "int64.onnx")
    t = pb_field(1, 0, pb_varint(2)) + pb_field(2, 0, pb_varint(7)) + pb_field(8, 2, b"i")
    open(bad_type, "wb").write(pb_field(7, 2, pb_field(5, 2, t)))
    expect_error(lambda: host.load_onnx_weights(bad_type), "invalid_argument", "7")
    size = str(tmp_path / "size.onnx")
    t = pb_field(1, 0, pb_varint(4)) + pb_field(2, 0, pb_varint(1)) + pb_field(8, 2, b"s") + pb_field(9, 2, b"\0" * 12)
    open(size, "wb").write(pb_field(7, 2, pb_field(5, 2, t)))
    expect_error(lambda: host.load_onnx_weights(size), "invalid_argument", "s")
    nograph = str(tmp_path / "nograph.onnx")
    open(nograph, "wb").write(pb_field(1, 0, pb_varint(8)))
    expect_error(lambda: host.load_onnx_weights(nograph), "invalid_argument", "graph")
    expect_error(lambda: host.save_onnx_weights(str(tmp_path / "i.onnx"), {"i": (I32, np.zeros(3, np.int32))}),
                 "invalid_argument", "i")
    expect_error(lambda: host.save_onnx_weights(str(tmp_path / "no_dir" / "x.onnx"), weights()), "invalid_argument")


def test_save_rejects_null_name_null_data_and_bad_dtype(tmp_path):
    """frame_save_onnx_weights checks each entry before reading it: a null name, null data for a non-empty tensor
    and a dtype code other than float32 / float16 / bfloat16 are invalid arguments (code 1) that write no file."""
    import ctypes
    lib = host.lib()
    path = str(tmp_path / "bad.onnx")
    data = np.arange(4, dtype=np.float32)
    dims = (ctypes.c_int64 * 1)(4)
    dims_pp = (ctypes.c_void_p * 1)(ctypes.cast(dims, ctypes.c_void_p))
    ranks = (ctypes.c_int32 * 1)(1)
    good_name = (ctypes.c_char_p * 1)(b"w")
    null_name = (ctypes.c_char_p * 1)(None)
    good_data = (ctypes.c_void_p * 1)(data.ctypes.data)
    null_data = (ctypes.c_void_p * 1)(None)
    for names, dtype, ptrs, what in ((null_name, F32, good_data, "null name"), (good_name, F32, null_data, "null data"),
                                     (good_name, I32, good_data, "int32"), (good_name, 17, good_data, "code 17")):
        dt = (ctypes.c_int32 * 1)(dtype)
        rc = lib.frame_save_onnx_weights(path.encode(), 1, names, dt, dims_pp, ranks, ptrs)
        assert rc == 1, (what, rc)
        assert not os.path.exists(path), what
    dt = (ctypes.c_int32 * 1)(F32)
    assert lib.frame_save_onnx_weights(path.encode(), 1, good_name, dt, dims_pp, ranks, good_data) == 0
    assert os.path.exists(path)

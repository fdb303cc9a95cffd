"""Kernel-level parity: every C-ABI kernel of libframe_hip_kernels.so against the oracle on identical seeded
inputs. Tolerances are stated per test (criterion in tests/tolerance.py); data movement, max-pool selections
and single elementwise ops are compared bit-for-bit."""
import ctypes

import numpy as np
import pytest

import oracle_lib as orc
from frame_hip import synth
from tolerance import assert_bitwise, assert_close

pytestmark = pytest.mark.gpu

F32, F16, BF16 = 0, 2, 3


def say(msg):
    print(f"[case] {msg}", flush=True)


def dev(hip, a):
    return hip.to_device(np.ascontiguousarray(a))


def run_gemm(hip, dtype, a, b, epilogue_segments=None):
    m, k = a.shape
    n = b.shape[1]
    da, db = dev(hip, a), dev(hip, b)
    dc = hip.DeviceBuffer(m * n * a.itemsize)
    ep = None
    keep = []
    if epilogue_segments:
        segs = []
        for op, operand in epilogue_segments:
            if operand is None:
                segs.append((op, None))
            else:
                d = dev(hip, operand)
                keep.append(d)
                segs.append((op, d.value))
        ep = ctypes.byref(hip.make_epilogue(segs))
    hip.check(hip.lib().fh_gemm(dtype, da.value, db.value, dc.value, m, n, k, ep, None), "fh_gemm")
    hip.check(hip.lib().fh_device_synchronize())
    return dc.download((m, n), a.dtype)


GEMM_SHAPES = [
    (64, 784, 256),   # C1 layer 1 (tile kernel, guarded: 64 rows)
    (64, 256, 10),    # C1 layer 2 (generic kernel: N not a multiple of the chunk width)
    (128, 128, 128),
    (300, 264, 200),  # ragged: every edge guarded
    (1, 8, 8),
    (512, 64, 512),   # attention scores shape
    (512, 512, 64),   # attention context shape
    (17, 3, 4096),    # tiny N, long K
]


@pytest.mark.parametrize("dtype", [F32, BF16, F16])
@pytest.mark.parametrize("shape", GEMM_SHAPES)
def test_gemm_matches_oracle(hip, dtype, shape):
    m, k, n = shape
    say(f"gemm dtype={dtype} m={m} k={k} n={n}")
    a = synth.tensor(11, (m, k), dtype, "uniform")
    b = synth.tensor(12, (k, n), dtype, "uniform")
    got = run_gemm(hip, dtype, a, b)
    want = orc.matmul(dtype, a, b)
    assert_close(got, want, dtype, what=f"gemm {shape}")


# Small problems (fp32: fewer 64x64 tiles than a quarter of the CUs; 16-bit: fewer than 16) and unaligned operands
# run the sequential kernel: one output per thread with k summed in order in fp32, like the reference CPU
# kernel, so it matches bit for bit.
SEQ_SHAPES = [
    (64, 784, 256),   # C1 layer 1
    (64, 256, 10),    # C1 layer 2
    (128, 128, 128),
    (512, 512, 64),
    (1, 8, 8),
    (3, 1, 5),        # K = 1
    (7, 131, 3),      # K tail shorter than one 4-wide step
]
SEQ_SHAPES_F32_ONLY = [
    (64, 512, 1000),  # the C4 classifier shape (16 tiles: MFMA for 16-bit types)
    (300, 264, 200),  # ragged tiles (20 tiles)
]


@pytest.mark.parametrize("dtype,shape", [(d, s) for d in (F32, BF16, F16) for s in SEQ_SHAPES] +
                         [(F32, s) for s in SEQ_SHAPES_F32_ONLY])
def test_gemm_small_bit_exact(hip, dtype, shape):
    m, k, n = shape
    say(f"gemm small dtype={dtype} m={m} k={k} n={n}")
    a = synth.tensor(13, (m, k), dtype, "uniform")
    b = synth.tensor(14, (k, n), dtype, "uniform")
    assert_bitwise(run_gemm(hip, dtype, a, b), orc.matmul(dtype, a, b), f"small gemm {shape}")


def test_gemm_known_answer(hip):
    # reference: tests/cpp/ops/test_op_matmul.cpp:208-230 — [[1,2],[3,4]]·[[5,6],[7,8]] = [[19,22],[43,50]]
    a = np.array([[1, 2], [3, 4]], np.float32)
    b = np.array([[5, 6], [7, 8]], np.float32)
    got = run_gemm(hip, F32, a, b)
    assert_bitwise(got, np.array([[19, 22], [43, 50]], np.float32), "matmul known answer")


@pytest.mark.parametrize("dtype", [F32, BF16])
@pytest.mark.parametrize("n", [1024, 2048])
def test_gemm_square_full(hip, dtype, n):
    say(f"gemm square full dtype={dtype} n={n}")
    a = synth.tensor(21, (n, n), dtype, "uniform")
    b = synth.tensor(22, (n, n), dtype, "uniform")
    got = run_gemm(hip, dtype, a, b)
    if n <= 1024:
        want = orc.matmul(dtype, a, b)
        assert_close(got, want, dtype, what=f"gemm {n}")
    else:
        rng = np.random.default_rng(5)
        rows, cols = rng.integers(0, n, 4096), rng.integers(0, n, 4096)
        want = orc.matmul_sample(dtype, a, b, rows, cols)
        assert_close(got[rows, cols], want, dtype, what=f"gemm {n} sampled")


@pytest.mark.parametrize("dtype", [F32, BF16])
def test_gemm_4096_sampled(hip, dtype):
    n = 4096
    say(f"gemm 4096 sampled dtype={dtype}")
    a = synth.tensor(31, (n, n), dtype, "uniform")
    b = synth.tensor(32, (n, n), dtype, "uniform")
    got = run_gemm(hip, dtype, a, b)
    rng = np.random.default_rng(7)
    rows, cols = rng.integers(0, n, 4096), rng.integers(0, n, 4096)
    want = orc.matmul_sample(dtype, a, b, rows, cols)
    assert_close(got[rows, cols], want, dtype, what="gemm 4096 sampled")
    # size-independent property: C = A·B implies C·1 = A·(B·1); checked on 8 rows in float64
    ones = np.ones(n)
    af, bf, cf = (synth.to_float(x, dtype).astype(np.float64) for x in (a, b, got))
    lhs = cf[:8] @ ones
    rhs = af[:8] @ (bf @ ones)
    scale = np.abs(af[:8]) @ (np.abs(bf) @ ones)
    assert np.all(np.abs(lhs - rhs) <= 1e-2 * scale), "row-sum identity"


@pytest.mark.parametrize("dtype", [BF16, F16])
@pytest.mark.parametrize("n", [64, 96])
def test_gemm_many_workgroups_per_cu(hip, dtype, n):
    # N < 128 selects the 64x64 tile (one MFMA per k16 half); M = 65536 gives 1024 workgroups, four per CU.
    # Regression test for the post-loop fragment fence: the last step's LDS reads (inline asm) are still in flight
    # when the loop ends, and without the fence the compiler reused their destination registers for the first
    # epilogue values, which the landing reads then overwrote (a few hundred wrong outputs per run, varying from
    # run to run). Three runs must agree bit for bit and match the oracle.
    m, k = 65536, 256
    say(f"gemm many workgroups per CU dtype={dtype} m={m} k={k} n={n}")
    a = synth.tensor(51, (m, k), dtype, "uniform")
    b = synth.tensor(52, (k, n), dtype, "uniform")
    runs = [run_gemm(hip, dtype, a, b) for _ in range(3)]
    for r in runs[1:]:
        assert_bitwise(r, runs[0], "repeat runs")
    rows = np.arange(0, m, 7)
    want = orc.matmul(dtype, a[rows], b)
    assert_close(runs[0][rows], want, dtype, what="gemm many workgroups per CU")


@pytest.mark.parametrize("dtype", [F32, BF16])
def test_gemm_epilogue_add_relu(hip, dtype):
    # matmul -> add(bias[M,N]) -> relu, as Frame's Linear + fused add;relu computes it (rounded between segments)
    m, k, n = 256, 192, 512
    say(f"gemm epilogue add;relu dtype={dtype}")
    a = synth.tensor(41, (m, k), dtype, "normal")
    b = synth.tensor(42, (k, n), dtype, "normal", 0.1)
    bias = synth.tensor(43, (m, n), dtype, "normal")
    got = run_gemm(hip, dtype, a, b, [(hip.EW_ADD, bias), (hip.EW_RELU, None)])
    mm = orc.matmul(dtype, a, b)
    want = orc.ew_program(dtype, [1, 3], [2, 1], [mm, bias])
    assert_close(got, want, dtype, what="gemm epilogue")


# C5's O-projection and FFN-down shapes with bias and residual (add;add), add only, and ragged edges, on 128x128
# tiles (one round of 256 workgroups), checked against the oracle on sampled outputs.
@pytest.mark.parametrize("m,n,k,program", [
    (4096, 1024, 1024, "add;add"),   # C5 O-projection + bias + residual
    (4096, 1024, 4096, "add;add"),   # C5 FFN-down + bias + residual
    (2048, 2048, 512, "add"),
    (2000, 2000, 96, "add;add"),     # 16 x 16 tiles, the last row and column of tiles ragged
])
def test_gemm_single_round_epilogue_operands(hip, m, n, k, program):
    say(f"gemm single-round epilogue {program} {m}x{n}x{k}")
    a = synth.tensor(61, (m, k), BF16, "normal")
    b = synth.tensor(62, (k, n), BF16, "normal", 0.05)
    ins = [synth.tensor(63, (m, n), BF16, "normal"), synth.tensor(64, (m, n), BF16, "normal")]
    nops = 2 if program == "add;add" else 1
    got = run_gemm(hip, BF16, a, b, [(hip.EW_ADD, ins[i]) for i in range(nops)])
    rng = np.random.default_rng(11)
    rows = np.concatenate([rng.integers(0, m, 3000), np.full(64, m - 1)])
    cols = np.concatenate([rng.integers(0, n, 3000), rng.integers(0, n, 64)])
    mm = orc.matmul_sample(BF16, a, b, rows, cols)
    want = orc.ew_program(BF16, [1] * nops, [2] * nops, [mm] + [x[rows, cols] for x in ins[:nops]])
    assert_close(got[rows, cols], want, BF16, what=f"single-round epilogue {program}")


@pytest.mark.parametrize("n", [256, 2048, 4096])  # 64x64, 128x128 and 256x256 tiles
def test_gemm_add_gelu_every_bf16_input(hip, n):
    # A.B = 0, so the add;gelu epilogue's gelu input is the operand itself, and the operand holds every bf16 pattern
    # (both zeros, denormals, the table band's edges, infinities, NaN): the bf16 epilogue's gelu (a table over the
    # band 2^-9 <= |x| < 8, closed forms outside it) equals the oracle's fp32 formula bit for bit, NaN as NaN
    m, k = n, 32
    say(f"gemm add;gelu over every bf16 pattern, {m}x{n}")
    bias = np.resize(np.arange(65536, dtype=np.uint16), (m, n))
    zeros_a = np.zeros((m, k), np.uint16)
    zeros_b = np.zeros((k, n), np.uint16)
    got = run_gemm(hip, BF16, zeros_a, zeros_b, [(hip.EW_ADD, bias), (hip.EW_GELU, None)])
    want = orc.ew_program(BF16, [1, 5], [2, 1], [np.zeros((m, n), np.uint16), bias])
    nan_got = (got & 0x7FFF) > 0x7F80
    nan_want = (want & 0x7FFF) > 0x7F80
    assert np.array_equal(nan_got, nan_want), "NaN positions differ"
    assert_bitwise(np.where(nan_got, 0, got), np.where(nan_want, 0, want), "add;gelu over every bf16 input")


def run_gemm_ex(hip, dtype, a, b, epilogue_segments=None, flags=1):
    """fh_gemm_ex (flags 1 = FH_GEMM_ANY_ORDER)."""
    m, k = a.shape
    n = b.shape[1]
    da, db = dev(hip, a), dev(hip, b)
    dc = hip.DeviceBuffer(m * n * a.itemsize)
    keep, segs = [], []
    for op, operand in epilogue_segments or []:
        if operand is None:
            segs.append((op, None))
        else:
            keep.append(dev(hip, operand))
            segs.append((op, keep[-1].value))
    ep = ctypes.byref(hip.make_epilogue(segs)) if segs else None
    hip.check(hip.lib().fh_gemm_ex(dtype, da.value, db.value, dc.value, m, n, k, ep, flags, None), "fh_gemm_ex")
    hip.check(hip.lib().fh_device_synchronize())
    return dc.download((m, n), a.dtype)


# Small GEMMs with FH_GEMM_ANY_ORDER (what the host passes at opt_level >= 1) run the split-k kernel: k summed in
# four interleaved quarters per 256-k chunk, the quarters added in order. Within the rule against the oracle,
# deterministic, and its epilogue is exact (fused == plain split-k GEMM followed by the elementwise program).
SPLIT_SHAPES = [
    (64, 784, 256),   # C1 layer 1
    (64, 256, 10),    # C1 layer 2
    (1, 8, 8),
    (100, 1000, 37),  # ragged rows, columns and chunks
    (4, 300, 16),
    (33, 5, 50),      # k below one wave's quarter
]


@pytest.mark.parametrize("dtype", [F32, BF16, F16])
@pytest.mark.parametrize("shape", SPLIT_SHAPES)
def test_gemm_split_k_matches_oracle(hip, dtype, shape):
    m, k, n = shape
    say(f"split-k gemm dtype={dtype} m={m} k={k} n={n}")
    a = synth.tensor(61, (m, k), dtype, "normal")
    b = synth.tensor(62, (k, n), dtype, "normal", 0.1)
    bias = synth.tensor(63, (m, n), dtype, "normal")
    got = run_gemm_ex(hip, dtype, a, b)
    assert_close(got, orc.matmul(dtype, a, b), dtype, what=f"split-k gemm {shape}")
    assert_bitwise(run_gemm_ex(hip, dtype, a, b), got, "split-k gemm, second call")
    fused = run_gemm_ex(hip, dtype, a, b, [(hip.EW_ADD, bias), (hip.EW_RELU, None)])
    assert_bitwise(fused, run_ew(hip, dtype, [1, 3], [2, 1], [got, bias]), "split-k epilogue vs separate program")


@pytest.mark.parametrize("dtype", [F32, BF16, F16])
@pytest.mark.parametrize("shape", [(64, 256, 10), (7, 40, 16), (300, 1500, 3)])
def test_gemm_row_softmax(hip, dtype, shape):
    """FH_GEMM_ROW_SOFTMAX: the split-k GEMM with its bias epilogue, then softmax over each row, in one launch;
    against the split-k GEMM alone followed by the oracle's softmax (and the oracle end to end)."""
    m, k, n = shape
    say(f"gemm + row softmax dtype={dtype} m={m} k={k} n={n}")
    a = synth.tensor(91, (m, k), dtype, "normal")
    b = synth.tensor(92, (k, n), dtype, "normal", 0.1)
    bias = synth.tensor(93, (m, n), dtype, "normal")
    fused = run_gemm_ex(hip, dtype, a, b, [(hip.EW_ADD, bias)], flags=3)
    logits = run_gemm_ex(hip, dtype, a, b, [(hip.EW_ADD, bias)], flags=1)
    assert_close(fused, orc.softmax(dtype, logits), dtype, what="fused softmax vs softmax of the same logits")
    want = orc.softmax(dtype, orc.ew_program(dtype, [1], [2], [orc.matmul(dtype, a, b), bias]))
    assert_close(fused, want, dtype, what="gemm + bias + softmax vs oracle")


def test_gemm_row_softmax_argument_checks(hip):
    a = dev(hip, np.zeros((8, 32), np.float32))
    b = dev(hip, np.zeros((32, 17), np.float32))
    c = hip.DeviceBuffer(8 * 17 * 4)
    lib = hip.lib()
    assert lib.fh_gemm_ex(F32, a.value, b.value, c.value, 8, 17, 32, None, 3, None) == 1  # N > 16
    assert lib.fh_gemm_ex(F32, a.value, b.value, c.value, 8, 16, 32, None, 2, None) == 1  # without any-order
    assert b"FH_GEMM_ROW_SOFTMAX" in lib.fh_last_error()


def run_gemm_grouped(hip, dtype, a, bs, biases):
    m, k = a.shape
    n = bs[0].shape[1]
    g = len(bs)
    da = dev(hip, a)
    dbs = [dev(hip, b) for b in bs]
    dcs = [hip.DeviceBuffer(m * n * a.itemsize) for _ in range(g)]
    dbias = [dev(hip, x) for x in biases] if biases else []
    eps = (hip.Epilogue * g)()
    for i in range(g):
        if biases:
            eps[i] = hip.make_epilogue([(hip.EW_ADD, dbias[i].value)])
    bp = (ctypes.c_void_p * g)(*[d.value for d in dbs])
    cp = (ctypes.c_void_p * g)(*[d.value for d in dcs])
    hip.check(hip.lib().fh_gemm_grouped(dtype, da.value, g, bp, cp, m, n, k, eps, 1, None), "fh_gemm_grouped")
    hip.check(hip.lib().fh_device_synchronize())
    return [d.download((m, n), a.dtype) for d in dcs]


@pytest.mark.parametrize("dtype", [BF16, F16])
@pytest.mark.parametrize("shape,groups,with_bias", [((512, 256, 256), 3, True), ((256, 128, 512), 2, False),
                                                     ((300, 96, 264), 4, True), ((4096, 1024, 1024), 3, True)])
def test_gemm_grouped_equals_separate_gemms(hip, dtype, shape, groups, with_bias):
    """fh_gemm_grouped (C5's merged Q/K/V projections) against one fh_gemm per group: the same MFMA kernel
    family sums every output in the same k order, so the results agree bit for bit (every shape here has at least
    16 tiles of 64 x 64 per group, so the single GEMMs take the MFMA kernel too); small shapes also against the
    oracle."""
    m, k, n = shape
    say(f"grouped gemm dtype={dtype} m={m} k={k} n={n} groups={groups} bias={with_bias}")
    a = synth.tensor(71, (m, k), dtype, "uniform")
    bs = [synth.tensor(72 + i, (k, n), dtype, "uniform") for i in range(groups)]
    biases = [synth.tensor(80 + i, (m, n), dtype, "normal") for i in range(groups)] if with_bias else None
    got = run_gemm_grouped(hip, dtype, a, bs, biases)
    for i in range(groups):
        segs = [(hip.EW_ADD, biases[i])] if with_bias else None
        assert_bitwise(got[i], run_gemm(hip, dtype, a, bs[i], segs), f"group {i} vs fh_gemm")
        if m * n * k <= (1 << 24):
            want = orc.matmul(dtype, a, bs[i])
            if with_bias:
                want = orc.ew_program(dtype, [1], [2], [want, biases[i]])
            assert_close(got[i], want, dtype, what=f"group {i} vs oracle")


def run_ew(hip, dtype, ops, arities, ins):
    dins = [dev(hip, x) for x in ins]
    out = hip.DeviceBuffer(ins[0].nbytes)
    o = (ctypes.c_uint8 * len(ops))(*ops)
    ar = (ctypes.c_int8 * len(arities))(*arities)
    ptrs = (ctypes.c_void_p * len(dins))(*[d.value for d in dins])
    hip.check(hip.lib().fh_ew_program(dtype, len(ops), o, ar, ptrs, len(dins), out.value, ins[0].size, 1, None))
    hip.check(hip.lib().fh_device_synchronize())
    return out.download(ins[0].shape, ins[0].dtype)


@pytest.mark.parametrize("dtype", [F32, BF16, F16])
@pytest.mark.parametrize("numel", [1, 7, 4096, 100003])
def test_ew_programs_bitwise(hip, dtype, numel):
    say(f"ew dtype={dtype} numel={numel}")
    x = synth.tensor(51, (numel,), dtype)
    y = synth.tensor(52, (numel,), dtype)
    z = synth.tensor(53, (numel,), dtype)
    for ops, ar, ins in [([1], [2], [x, y]), ([2], [2], [x, y]), ([3], [1], [x]), ([1, 3], [2, 1], [x, y]),
                         ([1, 2, 3], [2, 2, 1], [x, y, z]), ([4, 1], [1, 2], [x, y])]:
        got = run_ew(hip, dtype, ops, ar, ins)
        want = orc.ew_program(dtype, ops, ar, ins)
        assert_bitwise(got, want, f"ew {ops}")


def test_ew_special_values(hip):
    # relu keeps NaN and -0.0 like std::max(x, 0.0f) (reference: src/backends/cpu/kernels/elementwise.cpp:323-330)
    x = np.array([np.nan, -0.0, 0.0, -1.5, 2.5, np.inf, -np.inf, 1e-40], np.float32)
    got = run_ew(hip, F32, [3], [1], [x])
    want = orc.ew_program(F32, [3], [1], [x])
    assert_bitwise(got, want, "relu special values")
    assert np.signbit(got[1]) and np.isnan(got[0])


@pytest.mark.parametrize("dtype", [F32, BF16])
def test_gelu(hip, dtype):
    x = synth.tensor(55, (50000,), dtype, "normal", 3.0)
    got = run_ew(hip, dtype, [5], [1], [x])
    want = orc.ew_program(dtype, [5], [1], [x])
    # erff differs between libm and the device library by at most a few float32 ulps
    assert_close(got, want, dtype, rtol=1e-5 if dtype == F32 else 1e-2, atol=1e-6, what="gelu")


# (BF16, 512, 512), (BF16, 33, 1024), (F16, 5, 2048), (F32, 7, 256 / 512 / 1024) take the 16-byte vector kernel
@pytest.mark.parametrize("dtype,rows,cols", [(F32, 64, 10), (BF16, 512, 512), (F32, 3, 3000), (BF16, 8, 1),
                                             (F32, 2, 2), (BF16, 33, 1024), (F16, 5, 2048), (F32, 7, 256),
                                             (F32, 7, 512), (F32, 7, 1024), (BF16, 65536, 512)])
def test_softmax(hip, dtype, rows, cols):
    say(f"softmax dtype={dtype} {rows}x{cols}")
    x = synth.tensor(61, (rows, cols), dtype, "normal", 2.0)
    dx, dy = dev(hip, x), hip.DeviceBuffer(x.nbytes)
    hip.check(hip.lib().fh_softmax_rows(dtype, dx.value, dy.value, rows, cols, None))
    got = dy.download(x.shape, x.dtype)
    want = orc.softmax(dtype, x)
    assert_close(got, want, dtype, atol=1e-7 if dtype == F32 else 1e-4, what="softmax")
    say(f"  bit-identical fraction {np.mean(got == want):.4f}")


@pytest.mark.parametrize("cols", [512, 200])  # the 16-byte vector kernel and the per-element one
def test_softmax_16bit_special_rows(hip, cols):
    # bf16 softmax on v_exp_f32 and e * (1 / s): rows whose results are exact keep the reference's values bit for
    # bit (one-hot rows, ties), and infinities / NaN give NaN where the reference's arithmetic does
    ninf, inf, nan = -np.inf, np.inf, np.nan
    rows = [np.full(cols, ninf) for _ in range(6)]
    rows[0][3] = 0.0                      # one finite entry: y = 1 there, 0 elsewhere
    rows[1][:] = ninf                     # all -inf: x - m = NaN everywhere
    rows[2][0], rows[2][1:] = inf, 0.0    # +inf: inf - inf = NaN, the sum is NaN
    rows[3][:] = 1.0                      # ties: 1 / cols each
    rows[3][5] = nan                      # NaN in the row: the max skips it, its e and the sum are NaN
    rows[4][:] = 0.0                      # all equal: exactly 1 / cols (a power of two for 512)
    rows[5][:2] = 7.0                     # two equal maxima among -inf: 0.5 each
    x = synth.to_storage(np.stack(rows).astype(np.float32), BF16)
    dx, dy = dev(hip, x), hip.DeviceBuffer(x.nbytes)
    hip.check(hip.lib().fh_softmax_rows(BF16, dx.value, dy.value, len(rows), cols, None))
    got = dy.download(x.shape, x.dtype)
    want = orc.softmax(BF16, x)
    nan_got, nan_want = (got & 0x7FFF) > 0x7F80, (want & 0x7FFF) > 0x7F80
    assert np.array_equal(nan_got, nan_want), "NaN positions"
    assert_bitwise(np.where(nan_got, 0, got), np.where(nan_want, 0, want), "softmax special rows")


def test_softmax_known_answer(hip):
    # reference: tests/cpp/ops/test_op_softmax.cpp:123-162
    x = np.array([[1, 2], [3, 4]], np.float32)
    dx, dy = dev(hip, x), hip.DeviceBuffer(x.nbytes)
    hip.check(hip.lib().fh_softmax_rows(F32, dx.value, dy.value, 2, 2, None))
    got = dy.download((2, 2), np.float32)
    np.testing.assert_allclose(got, [[0.26894142, 0.73105858]] * 2, rtol=1e-6)


# (BF16, 4096, 1024), (BF16, 5, 512), (F16, 9, 2048), (F32, 6, 256/1024/2048) take the 16-byte vector kernel
@pytest.mark.parametrize("dtype,rows,cols", [(F32, 2, 5), (BF16, 4096, 1024), (F32, 3, 5000), (BF16, 7, 33),
                                             (BF16, 5, 512), (F16, 9, 2048), (F32, 6, 256), (F32, 6, 1024),
                                             (F32, 3, 2048)])
def test_layer_norm(hip, dtype, rows, cols):
    say(f"layer_norm dtype={dtype} {rows}x{cols}")
    x = synth.tensor(71, (rows, cols), dtype, "normal")
    g = synth.tensor(72, (cols,), dtype, "normal")
    b = synth.tensor(73, (cols,), dtype, "normal")
    dx, dg, db, dy = dev(hip, x), dev(hip, g), dev(hip, b), hip.DeviceBuffer(x.nbytes)
    hip.check(hip.lib().fh_layer_norm_rows(dtype, dx.value, dg.value, db.value, dy.value, rows, cols, 1e-5, None))
    got = dy.download(x.shape, x.dtype)
    want = orc.layer_norm(dtype, x, g, b, 1e-5)
    assert_close(got, want, dtype, what="layer_norm")
    say(f"  bit-identical fraction {np.mean(got == want):.4f}")


@pytest.mark.parametrize("dtype", [F32, BF16])
@pytest.mark.parametrize("mode,geom", [
    (0, (2, 3, 17, 17, 3, 3, 2, 2, 1, 1)),     # ResNet stem max-pool geometry, small
    (0, (1, 2, 9, 9, 3, 3, 2, 2, 1, 1)),
    (1, (2, 8, 7, 7, 7, 7, 1, 1, 0, 0)),       # global average pool
    (1, (1, 2, 6, 6, 3, 3, 2, 2, 1, 1)),       # average with padding counted
    (0, (2, 35000, 2, 2, 2, 2, 2, 2, 0, 0)),   # 70,000 planes: grid rows split over y and z
    (1, (1, 65537, 2, 2, 2, 2, 2, 2, 0, 0)),   # a prime plane count above 65,535: the general kernel
    (0, (1, 3, 300, 290, 3, 3, 2, 2, 1, 1)),   # planes spanning several 256-output blocks
    (0, (2, 4, 32, 32, 3, 3, 2, 2, 1, 1)),     # 16-bit: the vectorized 3x3 stride-2 kernel
    (0, (1, 3, 17, 48, 3, 3, 2, 2, 1, 1)),     # same, odd height: the last window's bottom row is padding
    (1, (2, 64, 7, 7, 7, 7, 1, 1, 0, 0)),      # global average pool, many planes
])
def test_pool2d(hip, dtype, mode, geom):
    say(f"pool mode={mode} dtype={dtype} {geom}")
    n, c, h, w = geom[:4]
    x = synth.tensor(81, (n, c, h, w), dtype, "normal")
    want = orc.pool2d(dtype, mode, x, geom)
    dx, dy = dev(hip, x), hip.DeviceBuffer(want.nbytes)
    hip.check(hip.lib().fh_pool2d(dtype, mode, dx.value, dy.value, hip.i64_array(geom), None))
    got = dy.download(want.shape, want.dtype)
    assert_bitwise(got, want, f"pool mode={mode}")


def test_maxpool_ties_and_neg_inf_padding(hip):
    # first maximum wins; padding never selected (reference: tests/cpp/ops/test_pool2d.cpp:361-600)
    x = np.full((1, 1, 4, 4), -5.0, np.float32)
    x[0, 0, 1, 1] = 7.0
    x[0, 0, 2, 2] = 7.0
    geom = (1, 1, 4, 4, 3, 3, 1, 1, 1, 1)
    want = orc.pool2d(F32, 0, x, geom)
    dx, dy = dev(hip, x), hip.DeviceBuffer(want.nbytes)
    hip.check(hip.lib().fh_pool2d(F32, 0, dx.value, dy.value, hip.i64_array(geom), None))
    assert_bitwise(dy.download(want.shape, np.float32), want, "maxpool ties")


@pytest.mark.parametrize("dtype", [BF16, F16])
def test_maxpool3s2_signed_zero_and_nan_selection(hip, dtype):
    # the vectorized 3x3 stride-2 kernel keeps the scan order: of equal +0/-0 the first stays, NaN first stays
    x = synth.tensor(85, (1, 2, 16, 32), dtype, "normal")
    neg0, pos0, nan = (synth.to_storage(np.array([v], np.float32), dtype)[0] for v in (-0.0, 0.0, np.nan))
    x[0, 0] = pos0
    x[0, 0, 0::2, 0::2] = neg0        # window origins -0: later +0 must not replace them
    x[0, 1, :4, :4] = nan             # NaN scanned first in its windows
    x[0, 1, 5, 7] = nan
    geom = (1, 2, 16, 32, 3, 3, 2, 2, 1, 1)
    want = orc.pool2d(dtype, 0, x, geom)
    dx, dy = dev(hip, x), hip.DeviceBuffer(want.nbytes)
    hip.check(hip.lib().fh_pool2d(dtype, 0, dx.value, dy.value, hip.i64_array(geom), None))
    assert_bitwise(dy.download(want.shape, want.dtype), want, "maxpool3s2 ties")


def test_permute_copy_fill(hip):
    x = np.arange(2 * 3 * 4 * 5, dtype=np.uint16).reshape(2, 3, 4, 5)
    for perm in [(1, 0, 2, 3), (0, 2, 1, 3), (3, 2, 1, 0)]:
        want = np.ascontiguousarray(np.transpose(x, perm))
        in_strides = np.array(x.strides) // x.itemsize
        dx, dy = dev(hip, x), hip.DeviceBuffer(x.nbytes)
        hip.check(hip.lib().fh_permute(2, dx.value, dy.value, 4, hip.i64_array(want.shape),
                                       hip.i64_array([in_strides[p] for p in perm]), None))
        assert_bitwise(dy.download(want.shape, np.uint16), want, f"permute {perm}")
    # rank-2 tiled transpose
    t = synth.tensor(91, (512, 64), BF16)
    dx, dy = dev(hip, t), hip.DeviceBuffer(t.nbytes)
    hip.check(hip.lib().fh_permute(2, dx.value, dy.value, 2, hip.i64_array([64, 512]), hip.i64_array([1, 64]), None))
    assert_bitwise(dy.download((64, 512), np.uint16), np.ascontiguousarray(t.T), "transpose2d")
    # column slice [512,1024] -> [512,64] at column 128 through copy2d
    s = synth.tensor(92, (512, 1024), BF16)
    ds, dd = dev(hip, s), hip.DeviceBuffer(512 * 64 * 2)
    hip.check(hip.lib().fh_copy2d(dd.value, 128, ds.value + 128 * 2, 2048, 128, 512, None))
    assert_bitwise(dd.download((512, 64), np.uint16), np.ascontiguousarray(s[:, 128:192]), "copy2d slice")
    # fill
    dfb = hip.DeviceBuffer(1000 * 2)
    hip.check(hip.lib().fh_fill(dfb.value, 2, 0x3E00, 1000, None))
    assert np.all(dfb.download((1000,), np.uint16) == 0x3E00)


CONV_CASES = [
    # N, Cin, H, W, Cout, KH, KW, sh, sw, ph, pw, groups, bias
    ((2, 3, 9, 9, 4, 7, 7, 2, 2, 3, 3, 1), True),
    ((2, 8, 7, 7, 8, 3, 3, 1, 1, 1, 1, 1), True),
    ((2, 8, 7, 7, 8, 3, 3, 1, 1, 1, 1, 2), False),     # groups
    ((1, 16, 14, 14, 32, 1, 1, 2, 2, 0, 0, 1), False), # 1x1 stride-2 downsample
    ((2, 64, 12, 12, 64, 3, 3, 1, 1, 1, 1, 1), True),
]


@pytest.mark.parametrize("dtype", [F32, BF16])
@pytest.mark.parametrize("geom,with_bias", CONV_CASES)
def test_conv2d(hip, dtype, geom, with_bias):
    say(f"conv dtype={dtype} {geom} bias={with_bias}")
    n, cin, h, w, cout, kh, kw = geom[:7]
    groups = geom[11]
    x = synth.tensor(101, (n, cin, h, w), dtype, "normal")
    wt = synth.tensor(102, (cout, cin // groups, kh, kw), dtype, "normal", (2.0 / (cin // groups * kh * kw)) ** 0.5)
    bias = synth.tensor(103, (cout,), dtype, "normal", 0.1) if with_bias else None
    want = orc.conv2d(dtype, x, wt, bias, geom)
    dx, dw = dev(hip, x), dev(hip, wt)
    db = dev(hip, bias) if with_bias else None
    dy = hip.DeviceBuffer(want.nbytes)
    hip.check(hip.lib().fh_conv2d_fwd(dtype, dx.value, dw.value, db.value if db else None, dy.value,
                                      hip.i64_array(geom), None, None))
    got = dy.download(want.shape, want.dtype)
    assert_close(got, want, dtype, what=f"conv {geom}")


# paths: whole planes through LDS (rows * cols <= 8192: filters), 16-byte tiles (16-bit, rows and cols multiples
# of 8; full and partial tiles), element tiles (everything else, e.g. thin late-stage activations)
@pytest.mark.parametrize("itemsize,shape", [(2, (3, 64, 3136)), (2, (2, 72, 200)), (2, (5, 70, 9)), (4, (2, 33, 130)),
                                            (2, (64, 64, 9)), (4, (2, 96, 100)), (2, (2, 70, 130)),
                                            (2, (2, 512, 49)), (2, (3, 64, 128)), (4, (3, 512, 9))])
def test_transpose_batched(hip, itemsize, shape):
    b, r, c = shape
    say(f"transpose_batched itemsize={itemsize} {shape}")
    dt = np.uint16 if itemsize == 2 else np.uint32
    x = np.random.default_rng(3).integers(0, np.iinfo(dt).max, size=shape, dtype=dt)
    dx, dy = dev(hip, x), hip.DeviceBuffer(x.nbytes)
    hip.check(hip.lib().fh_transpose_batched(itemsize, dx.value, dy.value, b, r, c, None))
    got = dy.download((b, c, r), dt)
    assert_bitwise(got, np.ascontiguousarray(x.transpose(0, 2, 1)), "batched transpose")


@pytest.mark.parametrize("itemsize", [2, 4])
@pytest.mark.parametrize("shapes", [
    [(64, 64, 9), (128, 64, 1), (5, 33, 7)],     # a 7-wide plane and 33 channels: the per-plane LDS kernel
    [(64, 64, 9), (128, 64, 1), (512, 512, 9)],  # 16-bit 3x3 and 1x1 with Cin % 8 == 0: the 16-byte vector kernel
    [(3, 8, 9), (1, 8, 9), (7, 16, 1)],          # one or two 8-channel groups per plane
])
def test_transpose_planes_multi(hip, itemsize, shapes):
    # tensors of different batch and plane shape (filters of 3x3, 1x1 and other convs) in one launch
    say(f"transpose_planes_multi itemsize={itemsize} {shapes}")
    dt = np.uint16 if itemsize == 2 else np.uint32
    rng = np.random.default_rng(11)
    xs = [rng.integers(0, np.iinfo(dt).max, size=s, dtype=dt) for s in shapes]
    dxs = [dev(hip, x) for x in xs]
    dys = [hip.DeviceBuffer(x.nbytes) for x in xs]
    n = len(shapes)
    ptrs_in = (ctypes.c_void_p * n)(*[d.value for d in dxs])
    ptrs_out = (ctypes.c_void_p * n)(*[d.value for d in dys])
    b = (ctypes.c_int64 * n)(*[s[0] for s in shapes])
    r = (ctypes.c_int64 * n)(*[s[1] for s in shapes])
    c = (ctypes.c_int64 * n)(*[s[2] for s in shapes])
    hip.check(hip.lib().fh_transpose_planes_multi(itemsize, n, ptrs_in, ptrs_out, b, r, c, None))
    for x, d, s in zip(xs, dys, shapes):
        assert_bitwise(d.download((s[0], s[2], s[1]), dt), np.ascontiguousarray(x.transpose(0, 2, 1)), f"multi {s}")


NHWC_CASES = [
    # N, Cin, H, W, Cout, KH, KW, sh, sw, ph, pw, groups, bias
    ((2, 64, 12, 12, 64, 3, 3, 1, 1, 1, 1, 1), True),
    ((2, 64, 7, 7, 128, 3, 3, 1, 1, 1, 1, 1), True),      # Ho*Wo = 49: element stores
    ((1, 128, 14, 14, 256, 3, 3, 2, 2, 1, 1, 1), False),  # stride 2, Ho*Wo = 49
    ((2, 64, 14, 14, 128, 1, 1, 2, 2, 0, 0, 1), False),   # 1x1 stride-2 downsample
    ((1, 32, 9, 11, 40, 3, 5, 1, 2, 2, 0, 1), True),      # rectangular, Cout not a tile multiple
    ((3, 96, 8, 8, 64, 3, 3, 1, 1, 1, 1, 1), True),       # Cin = 3 stages per filter position
]


def to_nhwc(x):
    return np.ascontiguousarray(x.transpose(0, 2, 3, 1))


# fp32 takes Cin % 16 == 0 (16 channels of 4 bytes per stage): these only it accepts
NHWC_F32_CASES = [
    ((1, 16, 10, 10, 48, 3, 3, 1, 1, 1, 1, 1), True),
    ((2, 48, 7, 9, 64, 3, 3, 2, 1, 1, 1, 1), False),
]


@pytest.mark.parametrize("dtype,geom,with_bias",
                         [(d, g, b) for d in (BF16, F16, F32) for g, b in NHWC_CASES] +
                         [(F32, g, b) for g, b in NHWC_F32_CASES])
def test_conv2d_nhwc(hip, dtype, geom, with_bias):
    say(f"conv nhwc dtype={dtype} {geom} bias={with_bias}")
    n, cin, h, w, cout, kh, kw = geom[:7]
    assert hip.lib().fh_conv2d_nhwc_supported(dtype, hip.i64_array(geom)) == 1
    x = synth.tensor(111, (n, cin, h, w), dtype, "normal")
    wt = synth.tensor(112, (cout, cin, kh, kw), dtype, "normal", (2.0 / (cin * kh * kw)) ** 0.5)
    bias = synth.tensor(113, (cout,), dtype, "normal", 0.1) if with_bias else None
    want = orc.conv2d(dtype, x, wt, bias, geom)
    dx, dw = dev(hip, to_nhwc(x)), dev(hip, to_nhwc(wt))
    db = dev(hip, bias) if with_bias else None
    dy = hip.DeviceBuffer(want.nbytes)
    hip.check(hip.lib().fh_conv2d_nhwc_fwd(dtype, dx.value, dw.value, db.value if db else None, dy.value,
                                           hip.i64_array(geom), None, None))
    got = dy.download(want.shape, want.dtype)
    assert_close(got, want, dtype, what=f"conv nhwc {geom}")


# Shapes large enough for each tile configuration of the implicit-GEMM dispatch table (64x256, 64x128, 128x256,
# 128x128; the small cases above take 64x64; FH_CONV_IMPLICIT_GEMM keeps these 3x3 stride-1 convs off the
# resident-patch kernel), checked on 4,096 sampled outputs recomputed by the oracle's per-element formula (the
# full single-threaded oracle would take minutes here).
LARGE_NHWC_CASES = [
    (BF16, (8, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1)),     # 64x256
    (BF16, (4, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1)),     # 64x128
    (BF16, (32, 128, 28, 28, 128, 3, 3, 1, 1, 1, 1, 1)),  # 128x256
    (BF16, (64, 256, 14, 14, 256, 3, 3, 1, 1, 1, 1, 1)),  # 128x128
    (F32, (8, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1)),      # 64x256
    (F32, (32, 128, 28, 28, 128, 3, 3, 1, 1, 1, 1, 1)),   # 128x128 (no 128x256 for fp32)
]


@pytest.mark.parametrize("dtype,geom", LARGE_NHWC_CASES)
def test_conv2d_nhwc_large_tiles_sampled(hip, dtype, geom):
    say(f"conv nhwc large dtype={dtype} {geom}")
    n, cin, h, w, cout, kh, kw = geom[:7]
    x = synth.tensor(141, (n, cin, h, w), dtype, "normal")
    wt = synth.tensor(142, (cout, cin, kh, kw), dtype, "normal", (2.0 / (cin * kh * kw)) ** 0.5)
    bias = synth.tensor(143, (cout,), dtype, "normal", 0.1)
    oh, ow = orc.conv_out_hw(geom)
    dx, dw, db = dev(hip, to_nhwc(x)), dev(hip, to_nhwc(wt)), dev(hip, bias)
    dy = hip.DeviceBuffer(n * cout * oh * ow * x.itemsize)
    hip.check(hip.lib().fh_conv2d_nhwc_fwd_ex(dtype, dx.value, dw.value, db.value, dy.value, hip.i64_array(geom),
                                              None, 2, None))  # 2 = FH_CONV_IMPLICIT_GEMM
    got = dy.download((n, cout, oh, ow), x.dtype).reshape(-1)
    idx = np.random.default_rng(7).integers(0, got.size, 4096)
    want = orc.conv2d_sample(dtype, x, wt, bias, geom, idx)
    assert_close(got[idx], want, dtype, what=f"conv nhwc large {geom}")


# The resident-patch kernel (3x3, stride 1, padding 1, 16-bit, Cin % 32 == 0): 256-pixel tiles where they still
# fill the device, 128 otherwise; tiles that straddle images (7x7 and 14x14 planes hold several images per tile),
# Cout below and above the 64-channel tile, channels-last output with the residual epilogue; sampled outputs
# everywhere in the batch (first and last images included) plus the full first and last images.
HALO_CASES = [
    # NCHW output: the single-buffered kernel (two workgroups per CU)
    (BF16, (32, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1), 0),    # C3: 256-pixel tiles
    (F16, (32, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1), 0),
    (BF16, (3, 96, 9, 13, 40, 3, 3, 1, 1, 1, 1, 1), 0),      # Cout 40, odd plane, 128-pixel tiles
    # channels-last output with the residual add;relu, 64 < Cout <= 256: single-buffered, workgroup-wide staging
    (BF16, (16, 128, 28, 28, 128, 3, 3, 1, 1, 1, 1, 1), 1),
    (BF16, (64, 256, 14, 14, 256, 3, 3, 1, 1, 1, 1, 1), 1),
    (BF16, (8, 256, 7, 7, 256, 3, 3, 1, 1, 1, 1, 1), 1),     # ~2.6 images per tile
    (BF16, (5, 32, 3, 5, 100, 3, 3, 1, 1, 1, 1, 1), 1),      # Cout 100 over two channel tiles, 3-row images
    # channels-last output, Cout <= 64: the persistent kernel (filter resident when Cin <= 64)
    (BF16, (64, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1), 1),    # ResNet layer 1: 256-pixel tiles, two per CU
    (BF16, (4, 32, 10, 12, 48, 3, 3, 1, 1, 1, 1, 1), 1),     # one chunk, Cout 48, 128-pixel tiles
    (BF16, (6, 128, 14, 14, 64, 3, 3, 1, 1, 1, 1, 1), 1),    # Cin 128: filter streamed with each step
    (F16, (2, 64, 12, 12, 64, 3, 3, 1, 1, 1, 1, 1), 1),
]


@pytest.mark.parametrize("dtype,geom,nhwc_out", HALO_CASES)
def test_conv2d_resident_patch(hip, dtype, geom, nhwc_out):
    say(f"conv resident patch dtype={dtype} {geom} nhwc_out={nhwc_out}")
    n, cin, h, w, cout, kh, kw = geom[:7]
    x = synth.tensor(171, (n, cin, h, w), dtype, "normal")
    wt = synth.tensor(172, (cout, cin, kh, kw), dtype, "normal", (2.0 / (cin * kh * kw)) ** 0.5)
    bias = synth.tensor(173, (cout,), dtype, "normal", 0.1)
    res = synth.tensor(174, (n, cout, h, w), dtype, "normal") if nhwc_out else None
    dx, dw, db = dev(hip, to_nhwc(x)), dev(hip, to_nhwc(wt)), dev(hip, bias)
    dy = hip.DeviceBuffer(n * cout * h * w * x.itemsize)
    ep = None
    if nhwc_out:
        dr = dev(hip, to_nhwc(res))
        ep = hip.make_epilogue([(hip.EW_ADD, dr.value), (hip.EW_RELU, None)])
    hip.check(hip.lib().fh_conv2d_nhwc_fwd_ex(dtype, dx.value, dw.value, db.value, dy.value, hip.i64_array(geom),
                                              ctypes.byref(ep) if ep else None, nhwc_out, None))
    got = dy.download((n, h, w, cout) if nhwc_out else (n, cout, h, w), x.dtype)
    if nhwc_out:
        got = np.ascontiguousarray(got.transpose(0, 3, 1, 2))

    def expect(conv, r):
        return orc.ew_program(dtype, [1, 3], [2, 1], [conv, r]) if nhwc_out else conv

    for img in sorted({0, n - 1}):  # whole first and last images
        conv = orc.conv2d(dtype, x[img:img + 1], wt, bias, (1,) + geom[1:])
        assert_close(got[img:img + 1], expect(conv, res[img:img + 1] if nhwc_out else None), dtype,
                     what=f"resident patch {geom} image {img}")
    flat = got.reshape(-1)
    idx = np.random.default_rng(9).integers(0, flat.size, 4096)
    conv = orc.conv2d_sample(dtype, x, wt, bias, geom, idx)
    want = orc.ew_program(dtype, [1, 3], [2, 1], [conv, res.reshape(-1)[idx]]) if nhwc_out else conv
    assert_close(flat[idx], want, dtype, what=f"resident patch {geom} sampled")


NCHW_IN_CASES = [
    # NCHW output, Cin 64, Cout <= 64, bf16: the band kernel (whole output rows per workgroup, filter resident)
    (BF16, (32, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1), 0),    # C3: 7-row bands, 256 of them
    (F16, (32, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1), 0),     # f16: the single-buffered kernel
    (BF16, (16, 64, 32, 56, 64, 3, 3, 1, 1, 1, 1, 1), 0),    # 2-row bands
    (BF16, (256, 64, 16, 16, 64, 3, 3, 1, 1, 1, 1, 1), 0),   # whole-image bands: both halo rows zero, 4 waves idle
    (BF16, (64, 64, 8, 64, 40, 3, 3, 1, 1, 1, 1, 1), 0),     # Cout 40, W 64
    (BF16, (3, 64, 12, 40, 48, 3, 3, 1, 1, 1, 1, 1), 0),     # 1-row bands (fewer rows than CUs)
    (BF16, (128, 64, 12, 48, 64, 3, 3, 1, 1, 1, 1, 1), 0),   # 6-row bands of 9 tiles: the 9th split in channel halves
    # the single-buffered kernel
    (BF16, (3, 96, 9, 16, 40, 3, 3, 1, 1, 1, 1, 1), 0),      # Cout 40, three chunks, 128-pixel tiles
    (BF16, (5, 32, 3, 8, 100, 3, 3, 1, 1, 1, 1, 1), 1),      # 3-row images, one 8-pixel group per row
    (BF16, (4, 64, 14, 24, 64, 3, 3, 1, 1, 1, 1, 1), 1),     # channels-last output from NCHW input
    (BF16, (2, 64, 7, 8, 320, 3, 3, 1, 1, 1, 1, 1), 1),      # Cout > 256 with channels-last output
]


@pytest.mark.parametrize("dtype,geom,nhwc_out", NCHW_IN_CASES)
def test_conv2d_nchw_input(hip, dtype, geom, nhwc_out):
    """FH_CONV_IN_NCHW: the single-buffered resident-patch kernel fills its patch from NCHW activations through
    registers. Same kernel, same k order as the channels-last input, so the two agree bit for bit; and both images
    at the ends of the batch against the oracle."""
    say(f"conv nchw input dtype={dtype} {geom} nhwc_out={nhwc_out}")
    n, cin, h, w, cout, kh, kw = geom[:7]
    assert hip.lib().fh_conv2d_nchw_in_supported(dtype, hip.i64_array(geom)) == 1
    x = synth.tensor(181, (n, cin, h, w), dtype, "normal")
    wt = synth.tensor(182, (cout, cin, kh, kw), dtype, "normal", (2.0 / (cin * kh * kw)) ** 0.5)
    bias = synth.tensor(183, (cout,), dtype, "normal", 0.1)
    dxn, dxc, dw, db = dev(hip, x), dev(hip, to_nhwc(x)), dev(hip, to_nhwc(wt)), dev(hip, bias)
    ep = hip.make_epilogue([(hip.EW_RELU, None)])
    outs = []
    for xin, flag in ((dxn, 4), (dxc, 0)):
        dy = hip.DeviceBuffer(n * cout * h * w * x.itemsize)
        hip.check(hip.lib().fh_conv2d_nhwc_fwd_ex(dtype, xin.value, dw.value, db.value, dy.value, hip.i64_array(geom),
                                                  ctypes.byref(ep), flag | nhwc_out, None))
        got = dy.download((n, h, w, cout) if nhwc_out else (n, cout, h, w), x.dtype)
        outs.append(np.ascontiguousarray(got.transpose(0, 3, 1, 2)) if nhwc_out else got)
    # with channels-last output, a channels-last input takes the persistent kernel for Cout <= 64 and the implicit
    # GEMM above 256; elsewhere both inputs run the same kernel
    if not (nhwc_out and (cout <= 64 or cout > 256)):
        assert_bitwise(outs[0], outs[1], f"NCHW vs channels-last input {geom}")
    else:
        assert_close(outs[0], outs[1], dtype, what=f"NCHW vs channels-last input {geom}")
    for img in sorted({0, n - 1}):
        conv = orc.conv2d(dtype, x[img:img + 1], wt, bias, (1,) + geom[1:])
        assert_close(outs[0][img:img + 1], orc.ew_program(dtype, [3], [1], [conv]), dtype,
                     what=f"NCHW input {geom} image {img}")


@pytest.mark.parametrize("geom", [(32, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1), (64, 64, 8, 64, 40, 3, 3, 1, 1, 1, 1, 1),
                                  (3, 64, 12, 40, 48, 3, 3, 1, 1, 1, 1, 1), (128, 64, 12, 48, 64, 3, 3, 1, 1, 1, 1, 1),
              # W = 8 bands of R = 32 and R = 52 rows: more padding slots (2 (R + 2) 8) than threads
              (256, 64, 32, 8, 64, 3, 3, 1, 1, 1, 1, 1), (256, 64, 52, 8, 64, 3, 3, 1, 1, 1, 1, 1)])
def test_conv2d_band_residual(hip, geom):
    """The band kernel (NCHW input and output) with the residual add;relu program and no bias: both images at the
    ends of the batch and 4,096 sampled outputs against the oracle."""
    say(f"conv band kernel add;relu {geom}")
    n, cin, h, w, cout, kh, kw = geom[:7]
    x = synth.tensor(191, (n, cin, h, w), BF16, "normal")
    wt = synth.tensor(192, (cout, cin, kh, kw), BF16, "normal", (2.0 / (cin * kh * kw)) ** 0.5)
    res = synth.tensor(193, (n, cout, h, w), BF16, "normal")
    dx, dw, dr = dev(hip, x), dev(hip, to_nhwc(wt)), dev(hip, res)
    dy = hip.DeviceBuffer(n * cout * h * w * 2)
    ep = hip.make_epilogue([(hip.EW_ADD, dr.value), (hip.EW_RELU, None)])
    hip.check(hip.lib().fh_conv2d_nhwc_fwd_ex(BF16, dx.value, dw.value, None, dy.value, hip.i64_array(geom),
                                              ctypes.byref(ep), 4, None))
    got = dy.download((n, cout, h, w), x.dtype)
    for img in sorted({0, n - 1}):
        conv = orc.conv2d(BF16, x[img:img + 1], wt, None, (1,) + geom[1:])
        want = orc.ew_program(BF16, [1, 3], [2, 1], [conv, res[img:img + 1]])
        assert_close(got[img:img + 1], want, BF16, what=f"band add;relu {geom} image {img}")
    flat = got.reshape(-1)
    idx = np.random.default_rng(11).integers(0, flat.size, 4096)
    conv = orc.conv2d_sample(BF16, x, wt, None, geom, idx)
    want = orc.ew_program(BF16, [1, 3], [2, 1], [conv, res.reshape(-1)[idx]])
    assert_close(flat[idx], want, BF16, what=f"band add;relu {geom} sampled")


BAND_GEOMS = [(32, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1), (16, 64, 32, 56, 64, 3, 3, 1, 1, 1, 1, 1),
              (256, 64, 16, 16, 64, 3, 3, 1, 1, 1, 1, 1), (64, 64, 8, 64, 40, 3, 3, 1, 1, 1, 1, 1),
              (3, 64, 12, 40, 48, 3, 3, 1, 1, 1, 1, 1), (128, 64, 12, 48, 64, 3, 3, 1, 1, 1, 1, 1),
              # W = 8 bands of R = 32 and R = 52 rows: more padding slots (2 (R + 2) 8) than threads
              (256, 64, 32, 8, 64, 3, 3, 1, 1, 1, 1, 1), (256, 64, 52, 8, 64, 3, 3, 1, 1, 1, 1, 1)]


@pytest.mark.parametrize("geom", BAND_GEOMS)
@pytest.mark.parametrize("program", ["none", "relu", "add;relu"])
def test_conv2d_band_filter_oihw(hip, geom, program):
    """FH_CONV_W_OIHW: the band kernel takes the filter in the graph's own [Cout,Cin,KH,KW] layout and transposes it
    in registers on its way into LDS. The LDS image and the k order are those of the channels-last filter, so the
    two agree bit for bit; the first image against the oracle as well."""
    say(f"conv band kernel OIHW filter {geom} {program}")
    n, cin, h, w, cout, kh, kw = geom[:7]
    lib = hip.lib()
    x = synth.tensor(201, (n, cin, h, w), BF16, "normal")
    wt = synth.tensor(202, (cout, cin, kh, kw), BF16, "normal", (2.0 / (cin * kh * kw)) ** 0.5)
    bias = None if program == "add;relu" else synth.tensor(203, (cout,), BF16, "normal", 0.1)
    res = synth.tensor(204, (n, cout, h, w), BF16, "normal")
    dx, dwo, dwc, dr = dev(hip, x), dev(hip, wt), dev(hip, to_nhwc(wt)), dev(hip, res)
    db = dev(hip, bias) if bias is not None else None
    segs = {"none": [], "relu": [(hip.EW_RELU, None)], "add;relu": [(hip.EW_ADD, dr.value), (hip.EW_RELU, None)]}
    ep = hip.make_epilogue(segs[program]) if segs[program] else None
    g = hip.i64_array(geom)
    assert lib.fh_conv2d_w_oihw_supported(BF16, g, ctypes.byref(ep) if ep else None) == 1
    outs = []
    for wbuf, flags in ((dwo, 4 | 8), (dwc, 4)):
        dy = hip.DeviceBuffer(n * cout * h * w * 2)
        hip.check(lib.fh_conv2d_nhwc_fwd_ex(BF16, dx.value, wbuf.value, db.value if db else None, dy.value, g,
                                            ctypes.byref(ep) if ep else None, flags, None))
        outs.append(dy.download((n, cout, h, w), x.dtype))
    assert_bitwise(outs[0], outs[1], f"OIHW vs channels-last filter {geom} {program}")
    conv = orc.conv2d(BF16, x[:1], wt, bias, (1,) + geom[1:])
    if program == "relu":
        conv = orc.ew_program(BF16, [3], [1], [conv])
    elif program == "add;relu":
        conv = orc.ew_program(BF16, [1, 3], [2, 1], [conv, res[:1]])
    assert_close(outs[0][:1], conv, BF16, what=f"band OIHW filter {geom} {program} image 0")


def test_conv2d_band_filter_oihw_rejections(hip):
    lib = hip.lib()
    c3 = (32, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1)
    n, cin, h, w, cout = c3[:5]
    dx, dw, dy = hip.DeviceBuffer(n * cin * h * w * 2), hip.DeviceBuffer(cout * cin * 9 * 2), \
        hip.DeviceBuffer(n * cout * h * w * 2)
    gelu = hip.make_epilogue([(hip.EW_GELU, None)])
    # FH_CONV_W_OIHW without FH_CONV_IN_NCHW, or with channels-last output: invalid argument
    for flags in (8, 8 | 4 | 1):
        assert lib.fh_conv2d_nhwc_fwd_ex(BF16, dx.value, dw.value, None, dy.value, hip.i64_array(c3), None, flags,
                                         None) == 1
    # a program without a band instance, f16, Cin 96: unimplemented, nothing launched
    assert lib.fh_conv2d_nhwc_fwd_ex(BF16, dx.value, dw.value, None, dy.value, hip.i64_array(c3), ctypes.byref(gelu),
                                     12, None) == 4
    assert lib.fh_conv2d_nhwc_fwd_ex(F16, dx.value, dw.value, None, dy.value, hip.i64_array(c3), None, 12, None) == 4
    g96 = (8, 96, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1)
    assert lib.fh_conv2d_nhwc_fwd_ex(BF16, dx.value, dw.value, None, dy.value, hip.i64_array(g96), None, 12,
                                     None) == 4


def test_conv2d_nchw_input_rejections(hip):
    lib = hip.lib()
    for geom in [(1, 64, 8, 12, 64, 3, 3, 1, 1, 1, 1, 1),     # W % 8 != 0
                 (1, 64, 8, 16, 64, 3, 3, 2, 2, 1, 1, 1),     # stride 2
                 (1, 48, 8, 16, 64, 3, 3, 1, 1, 1, 1, 1)]:    # Cin % 32 != 0
        g = hip.i64_array(geom)
        assert lib.fh_conv2d_nchw_in_supported(BF16, g) == 0, geom
        x = hip.DeviceBuffer(64 * 8 * 16 * 2)
        assert lib.fh_conv2d_nhwc_fwd_ex(BF16, x.value, x.value, None, x.value, g, None, 4, None) == 4  # unimplemented
    assert lib.fh_conv2d_nchw_in_supported(F32, hip.i64_array((1, 64, 8, 16, 64, 3, 3, 1, 1, 1, 1, 1))) == 0


NHWC_OUT_CASES = [
    (BF16, (2, 64, 12, 12, 64, 3, 3, 1, 1, 1, 1, 1)),
    (BF16, (2, 64, 14, 14, 128, 1, 1, 2, 2, 0, 0, 1)),    # 1x1 stride-2 downsample
    (BF16, (1, 32, 9, 11, 40, 3, 5, 1, 2, 2, 0, 1)),      # Cout 40: whole 8-channel vectors, 5 groups
    (BF16, (1, 32, 9, 9, 36, 3, 3, 1, 1, 1, 1, 1)),       # Cout 36: element stores
    (F32, (2, 48, 7, 9, 64, 3, 3, 2, 1, 1, 1, 1)),
]


@pytest.mark.parametrize("dtype,geom", NHWC_OUT_CASES)
def test_conv2d_nhwc_channels_last_output(hip, dtype, geom):
    # FH_CONV_OUT_NHWC: y [N,Ho,Wo,Cout] with the residual add;relu epilogue read channels-last as well
    say(f"conv nhwc-out dtype={dtype} {geom}")
    n, cin, h, w, cout, kh, kw = geom[:7]
    x = synth.tensor(151, (n, cin, h, w), dtype, "normal")
    wt = synth.tensor(152, (cout, cin, kh, kw), dtype, "normal", (2.0 / (cin * kh * kw)) ** 0.5)
    bias = synth.tensor(153, (cout,), dtype, "normal", 0.1)
    conv = orc.conv2d(dtype, x, wt, bias, geom)
    res = synth.tensor(154, conv.shape, dtype, "normal")
    want = to_nhwc(orc.ew_program(dtype, [1, 3], [2, 1], [conv, res]))
    dx, dw, db, dr = dev(hip, to_nhwc(x)), dev(hip, to_nhwc(wt)), dev(hip, bias), dev(hip, to_nhwc(res))
    dy = hip.DeviceBuffer(want.nbytes)
    ep = hip.make_epilogue([(hip.EW_ADD, dr.value), (hip.EW_RELU, None)])
    hip.check(hip.lib().fh_conv2d_nhwc_fwd_ex(dtype, dx.value, dw.value, db.value, dy.value, hip.i64_array(geom),
                                              ctypes.byref(ep), 1, None))
    got = dy.download(want.shape, want.dtype)
    assert_close(got, want, dtype, what=f"conv nhwc-out {geom}")


@pytest.mark.parametrize("dtype", [BF16, F32])
@pytest.mark.parametrize("mode,geom", [
    (0, (2, 64, 16, 16, 3, 3, 2, 2, 1, 1)),   # ResNet stem pool, channels-last
    (1, (2, 64, 7, 7, 7, 7, 1, 1, 0, 0)),     # global average pool
    (0, (1, 12, 9, 9, 3, 3, 2, 2, 1, 1)),     # C not a multiple of the vector width: one channel per lane
    (1, (1, 16, 6, 6, 3, 3, 2, 2, 1, 1)),     # average with padding counted
    (0, (1, 16, 12, 12, 10, 10, 1, 1, 0, 0)), # window rows wider than one batch of 8 loads
    (1, (1, 24, 12, 12, 10, 9, 1, 1, 1, 0)),
    (0, (2, 8, 17, 15, 3, 3, 2, 2, 1, 1)),    # 3-wide rows (the fixed-width kernel), odd sizes: padded edges
    # whole-plane windows (the whole-plane kernel: a channel pair per thread, all positions loaded first)
    (1, (64, 512, 7, 7, 7, 7, 1, 1, 0, 0)),   # C4's global average pool
    (0, (3, 10, 5, 5, 5, 5, 1, 1, 0, 0)),     # global max
    (1, (2, 6, 8, 8, 8, 8, 1, 1, 0, 0)),      # 64 positions, the most the kernel holds
    (1, (2, 6, 9, 9, 9, 9, 1, 1, 0, 0)),      # 81 positions: the general kernel
    (1, (3, 7, 4, 4, 4, 4, 1, 1, 0, 0)),      # odd C: 16-bit pairs do not divide it, the general kernel
])
def test_pool2d_nhwc(hip, dtype, mode, geom):
    say(f"pool nhwc mode={mode} dtype={dtype} {geom}")
    n, c, h, w = geom[:4]
    x = synth.tensor(161, (n, c, h, w), dtype, "normal")
    want = to_nhwc(orc.pool2d(dtype, mode, x, geom))
    dx, dy = dev(hip, to_nhwc(x)), hip.DeviceBuffer(want.nbytes)
    hip.check(hip.lib().fh_pool2d_nhwc(dtype, mode, dx.value, dy.value, hip.i64_array(geom), None))
    assert_bitwise(dy.download(want.shape, want.dtype), want, f"pool nhwc mode={mode}")


@pytest.mark.parametrize("dtype", [BF16, F16])
def test_maxpool_nhwc_signed_zero_and_nan_selection(hip, dtype):
    # the channels-last 3x3 stride-2 kernel keeps the reference's scan order: of equal +0/-0 the first stays, a
    # NaN stays only where it is scanned first, otherwise the comparisons skip it
    geom = (1, 16, 10, 12, 3, 3, 2, 2, 1, 1)
    x = synth.tensor(87, geom[:4], dtype, "normal")
    neg0, pos0, nan = (synth.to_storage(np.array([v], np.float32), dtype)[0] for v in (-0.0, 0.0, np.nan))
    x[0, :8] = pos0
    x[0, :8, 0::2, 0::2] = neg0
    x[0, 8:, 3, 5] = nan
    x[0, 8:, 0, 0] = nan
    want = to_nhwc(orc.pool2d(dtype, 0, x, geom))
    dx, dy = dev(hip, to_nhwc(x)), hip.DeviceBuffer(want.nbytes)
    hip.check(hip.lib().fh_pool2d_nhwc(dtype, 0, dx.value, dy.value, hip.i64_array(geom), None))
    assert_bitwise(dy.download(want.shape, want.dtype), want, "maxpool nhwc special values")


@pytest.mark.parametrize("n,c,hw", [(3, 3, 224 * 8), (2, 1, 64), (1, 8, 40), (2, 3, 50), (1, 5, 7), (4, 3, 300),
                                    (2, 3, 224 * 224), (1, 7, 1028), (3, 2, 4)])  # a whole 224x224 plane, odd C
def test_conv_pack_input_c8(hip, n, c, hw):
    # [N][C][HW] -> [N][HW][8] with channels C..7 zero (one pixel per thread, the image from the grid's y)
    say(f"pack input c8 n={n} c={c} hw={hw}")
    x = np.random.default_rng(hw + c).integers(0, 65536, size=(n, c, hw), dtype=np.uint16)
    want = np.zeros((n, hw, 8), np.uint16)
    want[:, :, :c] = x.transpose(0, 2, 1)
    dx, dy = dev(hip, x), hip.DeviceBuffer(want.nbytes)
    hip.check(hip.lib().fh_conv_pack_input_c8(dx.value, dy.value, n, c, hw, None))
    assert_bitwise(dy.download(want.shape, np.uint16), want, "pack c8")


@pytest.mark.parametrize("dtype", [BF16, F32])
def test_conv2d_nhwc_epilogue_add_relu(hip, dtype):
    # conv + bias, then the residual add;relu of a ResNet basic block, rounded between segments
    geom = (2, 64, 14, 14, 64, 3, 3, 1, 1, 1, 1, 1)
    say(f"conv nhwc epilogue add;relu dtype={dtype}")
    x = synth.tensor(121, geom[:4], dtype, "normal")
    wt = synth.tensor(122, (64, 64, 3, 3), dtype, "normal", (2.0 / 576) ** 0.5)
    bias = synth.tensor(123, (64,), dtype, "normal", 0.1)
    res = synth.tensor(124, (2, 64, 14, 14), dtype, "normal")
    conv = orc.conv2d(dtype, x, wt, bias, geom)
    want = orc.ew_program(dtype, [1, 3], [2, 1], [conv, res])
    dx, dw, db, dr = dev(hip, to_nhwc(x)), dev(hip, to_nhwc(wt)), dev(hip, bias), dev(hip, res)
    dy = hip.DeviceBuffer(want.nbytes)
    ep = hip.make_epilogue([(hip.EW_ADD, dr.value), (hip.EW_RELU, None)])
    hip.check(hip.lib().fh_conv2d_nhwc_fwd(dtype, dx.value, dw.value, db.value, dy.value, hip.i64_array(geom),
                                           ctypes.byref(ep), None))
    got = dy.download(want.shape, want.dtype)
    assert_close(got, want, dtype, what="conv nhwc epilogue")


SPLIT_CASES = [
    # geometry, splits (0: the planned count), epilogue
    ((64, 512, 7, 7, 512, 3, 3, 1, 1, 1, 1, 1), 0, "add;relu"),  # ResNet-18 layer 4 at batch 64 (planned: 2)
    ((64, 512, 7, 7, 512, 3, 3, 1, 1, 1, 1, 1), 0, "relu"),
    ((3, 512, 7, 7, 512, 3, 3, 1, 1, 1, 1, 1), 5, "add;relu"),   # 147 pixels (a ragged 128-pixel tile), 144 / 5
    ((2, 256, 9, 7, 384, 3, 3, 2, 1, 1, 0, 1), 3, "none"),       # stride 2 x 1, asymmetric padding, no bias
    ((1, 64, 5, 5, 128, 1, 1, 1, 1, 0, 0, 1), 2, "add;add"),      # 2 k stages, one per split; the interpreter
]


@pytest.mark.parametrize("geom,splits,program", SPLIT_CASES)
def test_conv2d_nhwc_split_k(hip, geom, splits, program):
    # fh_conv2d_nhwc_fwd_split: fp32 partials per K range, summed in split order by the reduction, which adds the
    # bias, rounds once and runs the epilogue; checked against the oracle at 1e-2 and against the unsplit kernel
    say(f"conv split-K {geom} splits={splits} {program}")
    dtype = BF16
    n, cin, h, w, cout, kh, kw = geom[:7]
    x = synth.tensor(171, (n, cin, h, w), dtype, "normal")
    wt = synth.tensor(172, (cout, cin, kh, kw), dtype, "normal", (2.0 / (cin * kh * kw)) ** 0.5)
    with_bias = program != "none"
    bias = synth.tensor(173, (cout,), dtype, "normal", 0.1) if with_bias else None
    conv = orc.conv2d(dtype, x, wt, bias, geom)
    res = synth.tensor(174, conv.shape, dtype, "normal")
    res2 = synth.tensor(175, conv.shape, dtype, "normal")
    ops = {"none": [], "relu": [hip.EW_RELU], "add;relu": [hip.EW_ADD, hip.EW_RELU], "add;add": [hip.EW_ADD, hip.EW_ADD]}[program]
    operands, arity, inputs = [conv], [], []
    dr, dr2 = dev(hip, to_nhwc(res)), dev(hip, to_nhwc(res2))
    for i, op in enumerate(ops):
        arity.append(2 if op == hip.EW_ADD else 1)
        if op == hip.EW_ADD:
            operands.append(res if len(operands) == 1 else res2)
            inputs.append((op, (dr if len(inputs) == 0 else dr2).value))
        else:
            inputs.append((op, None))
    want = to_nhwc(orc.ew_program(dtype, ops, arity, operands) if ops else conv)
    lib = hip.lib()
    g = hip.i64_array(geom)
    k = ctypes.c_int32(splits)
    ws = lib.fh_conv2d_nhwc_split_workspace(dtype, g, 1, ctypes.byref(k))
    oh, ow = want.shape[1:3]
    assert k.value >= 2 and ws == k.value * n * oh * ow * cout * 4, (ws, k.value)
    if splits == 0:
        assert k.value == 2, "the planned split of ResNet-18's layer 4 at batch 64 on 256 CUs"
    dx, dw = dev(hip, to_nhwc(x)), dev(hip, to_nhwc(wt))
    db = dev(hip, bias) if with_bias else None
    dws, dy, dy1 = hip.DeviceBuffer(ws), hip.DeviceBuffer(want.nbytes), hip.DeviceBuffer(want.nbytes)
    ep = hip.make_epilogue(inputs) if inputs else None
    epp = ctypes.byref(ep) if ep is not None else None
    hip.check(lib.fh_conv2d_nhwc_fwd_split(dtype, dx.value, dw.value, db.value if db else None, dy.value, g, epp, 1,
                                           k.value, dws.value, ws, None))
    hip.check(lib.fh_conv2d_nhwc_fwd_ex(dtype, dx.value, dw.value, db.value if db else None, dy1.value, g, epp, 1, None))
    got, unsplit = dy.download(want.shape, want.dtype), dy1.download(want.shape, want.dtype)
    assert_close(got, want, dtype, what=f"split-K conv {geom}")
    assert_close(got, unsplit, dtype, what=f"split-K vs unsplit {geom}")


def test_conv2d_nhwc_split_k_rejections(hip):
    lib = hip.lib()
    l4 = hip.i64_array((64, 512, 7, 7, 512, 3, 3, 1, 1, 1, 1, 1))
    k = ctypes.c_int32(0)
    for dtype, flags in [(F32, 1), (BF16, 0), (BF16, 3)]:  # fp32, NCHW output, with FH_CONV_IMPLICIT_GEMM
        k.value = 0
        assert lib.fh_conv2d_nhwc_split_workspace(dtype, l4, flags, ctypes.byref(k)) in (0, -1)
    k.value = 2
    assert lib.fh_conv2d_nhwc_split_workspace(BF16, hip.i64_array((64, 512, 7, 7, 192, 3, 3, 1, 1, 1, 1, 1)), 1,
                                              ctypes.byref(k)) == -1  # Cout % 128 != 0
    k.value = 0
    assert lib.fh_conv2d_nhwc_split_workspace(BF16, hip.i64_array((64, 256, 14, 14, 256, 3, 3, 1, 1, 1, 1, 1)), 1,
                                              ctypes.byref(k)) == 0 and k.value == 0  # layer 3 stays unsplit
    need = lib.fh_conv2d_nhwc_split_workspace(BF16, l4, 1, ctypes.byref(k))
    buf = hip.DeviceBuffer(need)
    # a workspace one float short, a misaligned workspace
    assert lib.fh_conv2d_nhwc_fwd_split(BF16, buf.value, buf.value, None, buf.value, l4, None, 1, 0, buf.value,
                                        need - 4, None) == 1
    assert lib.fh_conv2d_nhwc_fwd_split(BF16, buf.value, buf.value, None, buf.value, l4, None, 1, 0, buf.value + 8,
                                        need - 8, None) == 1
    # an explicit split count where split K does not apply (fp32); a planned count of 0 runs the unsplit kernels
    assert lib.fh_conv2d_nhwc_fwd_split(F32, buf.value, buf.value, None, buf.value, l4, None, 1, 2, buf.value,
                                        need, None) == 4


def test_conv2d_nhwc_rejects_unsupported(hip):
    # channel counts the stage width does not divide (and no C8 layout for fp32) and grouped convolutions stay
    # on the direct path
    for dtype, geom in [(BF16, (1, 3, 9, 9, 4, 3, 3, 1, 1, 1, 1, 1)), (BF16, (1, 64, 9, 9, 64, 3, 3, 1, 1, 1, 1, 2)),
                        (BF16, (1, 48, 9, 9, 64, 3, 3, 1, 1, 1, 1, 1)), (F32, (1, 24, 9, 9, 64, 3, 3, 1, 1, 1, 1, 1)),
                        (F32, (1, 8, 9, 9, 64, 3, 3, 1, 1, 1, 1, 1))]:
        assert hip.lib().fh_conv2d_nhwc_supported(dtype, hip.i64_array(geom)) == 0
        status = hip.lib().fh_conv2d_nhwc_fwd(dtype, None, None, None, None, hip.i64_array(geom), None, None)
        assert status == 4, status  # FH_UNIMPLEMENTED


C8_CASES = [
    # N, Cin, H, W, Cout, KH, KW, sh, sw, ph, pw, groups, bias — Cin <= 8 through the C8 layout
    ((2, 3, 32, 32, 64, 7, 7, 2, 2, 3, 3, 1), True),   # ResNet stem geometry at 32 px
    ((1, 3, 15, 17, 40, 3, 3, 1, 1, 1, 1, 1), True),   # Ho*Wo not a multiple of 8, Cout ragged
    ((2, 8, 9, 9, 64, 5, 5, 1, 1, 2, 2, 1), False),    # Cin exactly 8
    ((1, 1, 12, 12, 64, 2, 2, 2, 2, 0, 0, 1), True),   # KW < 4: several filter rows per stage
]


@pytest.mark.parametrize("dtype", [BF16, F16])
@pytest.mark.parametrize("geom,with_bias", C8_CASES)
def test_conv2d_c8(hip, dtype, geom, with_bias):
    say(f"conv c8 dtype={dtype} {geom} bias={with_bias}")
    n, cin, h, w, cout, kh, kw = geom[:7]
    g8 = list(geom)
    g8[1] = 8
    assert hip.lib().fh_conv2d_nhwc_supported(dtype, hip.i64_array(g8)) == 1
    x = synth.tensor(131, (n, cin, h, w), dtype, "normal")
    wt = synth.tensor(132, (cout, cin, kh, kw), dtype, "normal", (2.0 / (cin * kh * kw)) ** 0.5)
    bias = synth.tensor(133, (cout,), dtype, "normal", 0.1) if with_bias else None
    want = orc.conv2d(dtype, x, wt, bias, geom)
    k8 = hip.lib().fh_conv_c8_filter_k(kh, kw)
    dx, dw = dev(hip, x), dev(hip, wt)
    xp, wp = hip.DeviceBuffer(n * h * w * 8 * 2), hip.DeviceBuffer(cout * k8 * 2)
    hip.check(hip.lib().fh_conv_pack_input_c8(dx.value, xp.value, n, cin, h * w, None))
    hip.check(hip.lib().fh_conv_pack_filter_c8(dw.value, wp.value, cout, cin, kh, kw, None))
    # the packed layouts themselves, bit for bit
    xh = xp.download((n, h * w, 8), np.uint16)
    assert_bitwise(xh[:, :, :cin], np.ascontiguousarray(x.reshape(n, cin, h * w).transpose(0, 2, 1)), "packed input")
    assert not xh[:, :, cin:].any()
    wh = wp.download((cout, k8), np.uint16)
    ref_w = np.zeros((cout, k8), np.uint16)
    ref_w[:, :kh * kw * 8].reshape(cout, kh * kw, 8)[:, :, :cin] = wt.reshape(cout, cin, kh * kw).transpose(0, 2, 1)
    assert_bitwise(wh, ref_w, "packed filter")
    db = dev(hip, bias) if with_bias else None
    dy = hip.DeviceBuffer(want.nbytes)
    hip.check(hip.lib().fh_conv2d_nhwc_fwd(dtype, xp.value, wp.value, db.value if db else None, dy.value,
                                           hip.i64_array(g8), None, None))
    got = dy.download(want.shape, want.dtype)
    assert_close(got, want, dtype, what=f"conv c8 {geom}")


# ---- fused stem: conv 7x7/2 + bias + relu + max pool 3x3/2 -------------------------------------------------

STEM_CASES = [
    (2, 3, 224, 224),  # C4's stem, two images: pool 56 x 56, 8 strips, 16-byte row stores
    (3, 3, 32, 48),    # pool 8 x 12: the second strip ragged, element stores
    (2, 1, 40, 64),    # one channel
    (1, 2, 35, 16),    # odd height: the last pool window has two rows; two channels; one strip
    (2, 3, 30, 112),   # pool 8 x 28
]


def stem_oracle(dtype, x, w, bias, relu):
    n, cin, h, wd = x.shape
    geom = (n, cin, h, wd, 64, 7, 7, 2, 2, 3, 3, 1)
    y = orc.conv2d(dtype, x, w, bias, geom)
    if relu:
        y = orc.ew_program(dtype, [3], [1], [y])
    oh, ow = y.shape[2], y.shape[3]
    return orc.pool2d(dtype, 0, y, (n, 64, oh, ow, 3, 3, 2, 2, 1, 1))


@pytest.mark.parametrize("dtype", [BF16, F16])
@pytest.mark.parametrize("shape", STEM_CASES)
def test_conv2d_stem_pool(hip, dtype, shape):
    """fh_conv2d_stem_pool against the oracle's conv2d -> relu -> max_pool2d. The conv values differ from the
    oracle's sequential sums within the tolerance, so the pooled values are held to the same rule; the selection
    itself is exact (the test below checks it where the conv values are exact)."""
    n, cin, h, wd = shape
    say(f"stem conv+pool dtype={dtype} {shape}")
    geom, pool = hip.i64_array((n, cin, h, wd, 64, 7, 7, 2, 2, 3, 3, 1)), hip.i64_array((3, 3, 2, 2, 1, 1))
    assert hip.lib().fh_conv2d_stem_pool_supported(dtype, geom, pool) == 1
    x = synth.tensor(141, (n, cin, h, wd), dtype, "normal")
    w = synth.tensor(142, (64, cin, 7, 7), dtype, "normal", (2.0 / (cin * 49)) ** 0.5)
    bias = synth.tensor(143, (64,), dtype, "normal", 0.1)
    dx, dw, db = dev(hip, x), dev(hip, w), dev(hip, bias)  # held: the buffers must outlive the launch
    for relu in (1, 0):
        want = stem_oracle(dtype, x, w, bias, relu)
        dy = hip.DeviceBuffer(want.nbytes)
        hip.check(hip.lib().fh_conv2d_stem_pool(dtype, dx.value, dw.value, db.value, dy.value, geom, pool, relu, None))
        got = dy.download(want.shape, want.dtype)
        assert_close(got, want, dtype, what=f"stem {shape} relu={relu}")


def test_conv2d_stem_pool_selection_is_exact(hip):
    """Integer-valued operands (small integers in x, the filter and the bias: every product and partial sum is an
    integer below 2^24, exact in fp32) make the fp32 sums identical in any summation order, so both sides round the
    same value and the fused result must equal the oracle's conv -> relu -> max_pool2d bit for bit, including the NaN
    rule of the reference's scan (a NaN in the input makes NaN conv values; a window whose first valid element is
    NaN gives NaN, later NaNs are skipped)."""
    rng = np.random.default_rng(7)
    n, cin, h, wd = 2, 3, 36, 48
    xf = rng.integers(-3, 4, (n, cin, h, wd)).astype(np.float32)
    wf = rng.integers(-2, 3, (64, cin, 7, 7)).astype(np.float32)
    bf = rng.integers(-4, 5, (64,)).astype(np.float32)
    xf[0, 1, 10, 20] = np.nan  # NaN conv values around (5, 10) of image 0
    xf[1, 0, 0, 0] = np.nan    # at the image corner: windows whose first element is NaN
    x, w, b = (synth.to_storage(a, BF16) for a in (xf, wf, bf))
    geom, pool = hip.i64_array((n, cin, h, wd, 64, 7, 7, 2, 2, 3, 3, 1)), hip.i64_array((3, 3, 2, 2, 1, 1))
    dx, dw, db = dev(hip, x), dev(hip, w), dev(hip, b)  # held: the buffers must outlive the launch
    for relu in (1, 0):
        want = stem_oracle(BF16, x, w, b, relu)
        dy = hip.DeviceBuffer(want.nbytes)
        hip.check(hip.lib().fh_conv2d_stem_pool(BF16, dx.value, dw.value, db.value, dy.value, geom, pool, relu, None))
        got = dy.download(want.shape, want.dtype)
        # NaN positions must agree; the NaN's sign and payload are the matrix core's, not the CPU's
        gnan, wnan = np.isnan(synth.to_float(got, BF16)), np.isnan(synth.to_float(want, BF16))
        assert wnan.any() and (gnan == wnan).all(), f"relu={relu}: NaN positions differ at {np.count_nonzero(gnan != wnan)}"
        assert_bitwise(np.where(wnan, 0, got), np.where(wnan, 0, want), f"stem exact relu={relu}")


def test_conv2d_stem_pool_rejections(hip):
    lib = hip.lib()
    pool = hip.i64_array((3, 3, 2, 2, 1, 1))
    ok = (2, 3, 224, 224, 64, 7, 7, 2, 2, 3, 3, 1)
    assert lib.fh_conv2d_stem_pool_supported(BF16, hip.i64_array(ok), pool) == 1
    assert lib.fh_conv2d_stem_pool_supported(F32, hip.i64_array(ok), pool) == 0
    for k, v in [(1, 4), (4, 32), (5, 5), (7, 1), (9, 2), (3, 220), (3, 232), (11, 3)]:
        bad = list(ok)
        bad[k] = v
        assert lib.fh_conv2d_stem_pool_supported(BF16, hip.i64_array(bad), pool) == 0, (k, v)
    assert lib.fh_conv2d_stem_pool_supported(BF16, hip.i64_array(ok), hip.i64_array((2, 2, 2, 2, 0, 0))) == 0
    dx = hip.DeviceBuffer(16)
    assert lib.fh_conv2d_stem_pool(BF16, dx.value, dx.value, None, dx.value, hip.i64_array((2, 3, 224, 232, 64, 7, 7, 2,
                                                                                         2, 3, 3, 1)), pool, 1, None) == 4


# ---- fused attention ------------------------------------------------------------------------------------

def attention_oracle(dtype, q, k, v, batch, seq, heads, dh, scale_value=None):
    """The reference's per-(batch, head) decomposition (src/nn/layers.cpp:1014-1080) evaluated node by node
    with the oracle: matmul(Q_bh, K_bh^T) -> mul by the 1/sqrt(dh) splat -> softmax -> matmul(., V_bh)."""
    sv = 1.0 / np.sqrt(dh) if scale_value is None else scale_value
    scale = synth.to_storage(np.full((seq, seq), sv, np.float32), dtype)
    out = np.empty_like(q)
    for b in range(batch):
        rows = slice(b * seq, (b + 1) * seq)
        for h in range(heads):
            cols = slice(h * dh, (h + 1) * dh)
            qh = np.ascontiguousarray(q[rows, cols])
            kt = np.ascontiguousarray(k[rows, cols].T)
            vh = np.ascontiguousarray(v[rows, cols])
            s = orc.matmul(dtype, qh, kt)
            s = orc.ew_program(dtype, [2], [2], [s, scale])  # fh_ew_op 2 = mul
            out[rows, cols] = orc.matmul(dtype, orc.softmax(dtype, s), vh)
    return out


ATTENTION_CASES = [
    # dtype, batch, seq, heads, input std[, scale]: 1/sqrt(64) = 0.125 is a power of two, which the kernel
    # folds into the exponent; the cases with 0.1 take its general path (round(round(S) * scale)). bf16 with seq a
    # multiple of 128 runs the key-split kernel (two waves per 32 queries), the rest the unsplit one
    (BF16, 2, 64, 2, 1.0),    # one 64-key tile per wave half; score-row swizzle over 8 chunks
    (BF16, 1, 128, 3, 1.0),   # 16 chunks per score row
    (BF16, 2, 192, 2, 1.0),   # 24 chunks: not a multiple of 16
    (BF16, 1, 320, 1, 1.0),   # 40 chunks
    (BF16, 1, 512, 2, 1.0),   # the largest sequence (C5's)
    (BF16, 8, 512, 16, 1.0),  # C5's whole attention: 8 x 16 (batch, head) pairs, 512 tasks on 256 workgroups
    (BF16, 1, 384, 87, 1.0),  # 261 tasks on 131 workgroups: the last one runs a single task; no XCD remap
    (BF16, 3, 512, 30, 1.0, 0.1),  # 360 tasks on 180 workgroups, the general-scale path
    (BF16, 1, 256, 2, 3.0),   # wide score range: most probabilities underflow to 0
    (F16, 2, 256, 2, 1.0),
    (F16, 1, 512, 1, 0.5),
    (BF16, 1, 512, 2, 1.0, 0.1),
    (BF16, 2, 192, 1, 3.0, 0.1),
    (F16, 1, 320, 2, 1.0, 0.1),
]


@pytest.mark.parametrize("case", ATTENTION_CASES, ids=lambda c: "-".join(str(x) for x in c))
def test_attention_matches_decomposition(hip, case):
    dtype, batch, seq, heads, std = case[:5]
    scale_value = case[5] if len(case) > 5 else None
    dh = 64
    say(f"attention dtype={dtype} batch={batch} seq={seq} heads={heads} std={std} scale={scale_value}")
    assert hip.lib().fh_attention_supported(dtype, seq, dh) == 1
    shape = (batch * seq, heads * dh)
    q = synth.tensor(141, shape, dtype, "normal", std)
    k = synth.tensor(142, shape, dtype, "normal", std)
    v = synth.tensor(143, shape, dtype, "normal")
    want = attention_oracle(dtype, q, k, v, batch, seq, heads, dh, scale_value)
    dq, dk, dv = dev(hip, q), dev(hip, k), dev(hip, v)
    dout = hip.DeviceBuffer(want.nbytes)
    sv = 1.0 / np.sqrt(dh) if scale_value is None else scale_value
    scale = float(synth.to_float(synth.to_storage(np.array([sv], np.float32), dtype), dtype)[0])
    hip.check(hip.lib().fh_attention_fwd(dtype, dq.value, dk.value, dv.value, dout.value, batch, seq, heads, dh,
                                         scale, None), "fh_attention_fwd")
    got = dout.download(want.shape, want.dtype)
    stats = assert_close(got, want, dtype, what=f"attention b={batch} s={seq} h={heads}")
    same = float(np.mean(got == want))
    print(f"  bit-identical fraction {same:.4f}, max abs err {stats['max_abs']:.3g} (rms {stats['rms']:.3g})")


def test_attention_rejects_unsupported(hip):
    # shapes outside the kernel's envelope are refused without a launch
    for dtype, seq, dh in [(F32, 128, 64), (BF16, 128, 32), (BF16, 96, 64), (BF16, 576, 64), (BF16, 0, 64)]:
        assert hip.lib().fh_attention_supported(dtype, seq, dh) == 0
        rc = hip.lib().fh_attention_fwd(dtype, None, None, None, None, 1, seq, 1, dh, 0.125, None)
        assert rc != 0, (dtype, seq, dh)


# out[ci][a][b][co] = w[co][ci][K-1-a][K-1-b]; (100, 13, 3, 3) and (64, 64, 3, 3) take the LDS-tiled form (ragged
# and whole 64-channel tiles), (70, 9, 17, 17) f32 the gather form (its tile would need more than 64 KB of LDS)
@pytest.mark.parametrize("itemsize,shape", [(2, (100, 13, 3, 3)), (2, (64, 64, 3, 3)), (4, (33, 17, 1, 1)),
                                            (2, (512, 256, 3, 3)), (4, (70, 9, 17, 17)), (4, (70, 9, 11, 11)), (2, (8, 3, 7, 5))])
def test_conv_filter_flip(hip, itemsize, shape):
    say(f"conv_filter_flip itemsize={itemsize} {shape}")
    dt = np.uint16 if itemsize == 2 else np.uint32
    dtype = 3 if itemsize == 2 else 0
    w = np.random.default_rng(5).integers(0, np.iinfo(dt).max, size=shape, dtype=dt)
    dw, dout = dev(hip, w), hip.DeviceBuffer(w.nbytes)
    co, ci, kh, kw = shape
    hip.check(hip.lib().fh_conv_filter_flip(dtype, dw.value, dout.value, co, ci, kh, kw, None))
    want = np.ascontiguousarray(w[:, :, ::-1, ::-1].transpose(1, 2, 3, 0))
    assert_bitwise(dout.download((ci, kh, kw, co), dt), want, f"filter flip {shape}")


# the batched form: a training graph's mix (3x3 and 1x1, whole and ragged 64-channel tiles, a 7x7 and an empty
# filter), each output against the permutation and against a single fh_conv_filter_flip call, bit for bit
@pytest.mark.parametrize("itemsize", [2, 4])
def test_conv_filter_flip_multi(hip, itemsize):
    shapes = [(64, 64, 3, 3), (100, 13, 3, 3), (0, 8, 3, 3), (128, 64, 1, 1), (512, 256, 3, 3), (64, 3, 7, 7),
              (33, 17, 1, 1), (8, 3, 7, 5)]
    say(f"conv_filter_flip_multi itemsize={itemsize} {len(shapes)} filters")
    dt = np.uint16 if itemsize == 2 else np.uint32
    dtype = 3 if itemsize == 2 else 0
    rng = np.random.default_rng(6)
    ws = [rng.integers(0, np.iinfo(dt).max, size=sh, dtype=dt) for sh in shapes]
    dws = [dev(hip, w) if w.size else hip.DeviceBuffer(16) for w in ws]
    outs = [hip.DeviceBuffer(max(w.nbytes, 16)) for w in ws]
    n = len(shapes)
    wp = (ctypes.c_void_p * n)(*[d.value for d in dws])
    op = (ctypes.c_void_p * n)(*[d.value for d in outs])
    dims = (ctypes.c_int64 * (4 * n))(*[v for sh in shapes for v in sh])
    hip.check(hip.lib().fh_conv_filter_flip_multi(dtype, n, wp, op, dims, None))
    for w, dw, o, (co, ci, kh, kw) in zip(ws, dws, outs, shapes):
        if w.size == 0:
            continue
        want = np.ascontiguousarray(w[:, :, ::-1, ::-1].transpose(1, 2, 3, 0))
        got = o.download((ci, kh, kw, co), dt)
        assert_bitwise(got, want, f"filter flip multi {w.shape}")
        single = hip.DeviceBuffer(w.nbytes)
        hip.check(hip.lib().fh_conv_filter_flip(dtype, dw.value, single.value, co, ci, kh, kw, None))
        assert_bitwise(got, single.download((ci, kh, kw, co), dt), f"filter flip multi vs single {w.shape}")
    # rejected before any launch: more than FH_FLIP_MAX filters, a filter above FH_FLIP_MAX_TAPS taps
    assert hip.lib().fh_conv_filter_flip_multi(dtype, 33, wp, op, dims, None) != 0
    big = (ctypes.c_int64 * 4)(8, 8, 16, 16)
    assert hip.lib().fh_conv_filter_flip_multi(dtype, 1, wp, op, big, None) != 0

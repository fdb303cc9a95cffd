"""Parity criterion of the build, in the reference's form |a - e| <= atol + rtol * |e|
(reference: tests/cpp/common/tolerance.h:41-62, 127; NaN is never close).

rtol follows the north-star bar: 1e-5 for float32, 1e-2 for bfloat16 and float16. Outputs of long reductions
(K up to 4096) can sit near zero, where a purely relative bound is meaningless, so atol is scaled from the
expected output's rms: atol = rtol * rms(expected). Each test states its tolerance where it calls this.
"""
from __future__ import annotations

import numpy as np

RTOL = {0: 1e-5, 2: 1e-2, 3: 1e-2}


def assert_close(actual: np.ndarray, expected: np.ndarray, dtype: int, rtol: float | None = None,
                 atol: float | None = None, what: str = "") -> dict:
    from frame_hip.synth import to_float

    a = to_float(np.asarray(actual), dtype).astype(np.float64).ravel()
    e = to_float(np.asarray(expected), dtype).astype(np.float64).ravel()
    assert a.shape == e.shape, (what, a.shape, e.shape)
    rtol = RTOL[dtype] if rtol is None else rtol
    finite = np.isfinite(e)
    rms = float(np.sqrt(np.mean(e[finite] ** 2))) if finite.any() else 0.0
    if atol is None:
        atol = rtol * rms
    err = np.abs(a - e)
    ok = err <= atol + rtol * np.abs(e)
    # NaN in both at the same place counts as a match only when the caller asks for exact bit parity elsewhere.
    ok &= ~(np.isnan(a) | np.isnan(e))
    stats = {"max_abs": float(err[finite].max()) if finite.any() else 0.0, "rms": rms, "atol": atol, "rtol": rtol,
             "n": int(a.size)}
    if not ok.all():
        bad = np.flatnonzero(~ok)
        i = int(bad[0])
        raise AssertionError(f"{what}: {bad.size}/{a.size} elements outside tolerance (rtol={rtol}, atol={atol:.3g});"
                             f" first at {i}: actual={a[i]!r} expected={e[i]!r}")
    return stats


def assert_bitwise(actual: np.ndarray, expected: np.ndarray, what: str = "") -> None:
    a = np.ascontiguousarray(actual).view(np.uint8)
    e = np.ascontiguousarray(expected).view(np.uint8)
    assert a.shape == e.shape, (what, a.shape, e.shape)
    if not np.array_equal(a, e):
        raise AssertionError(f"{what}: outputs differ bitwise at {np.count_nonzero(a != e)} bytes")

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


def assert_deep_lowp(actual: np.ndarray, oracle_lowp: np.ndarray, reference_f32: np.ndarray, dtype: int,
                     mean_slack: float = 1.25, max_slack: float = 2.0, what: str = "") -> dict:
    """Criterion for deep bf16/f16 graphs (many layers, every intermediate rounded to the storage type).

    Two correct low-precision evaluations that accumulate in different orders differ by more than the per-op
    1e-2 bound once rounding differences compound over layers (measured on ResNet-18 at 64 px: the reference
    CPU backend's own bf16 logits are up to 1.8 % of the logit rms away from an fp32 evaluation). Both the
    result and the oracle's low-precision result are therefore compared with `reference_f32` — the same graph
    evaluated in float32 on the same (low-precision-valued) inputs. The result's mean absolute error may exceed
    the oracle's own by at most `mean_slack`; its maximum, a single-element statistic that varies by tens of
    percent between two equally correct evaluations (measured: 1.42x between them on ResNet-18 at 224 px with
    equal means), by at most `max_slack`.
    """
    from frame_hip.synth import to_float

    a = to_float(np.asarray(actual), dtype).astype(np.float64).ravel()
    o = to_float(np.asarray(oracle_lowp), dtype).astype(np.float64).ravel()
    f = np.asarray(reference_f32, dtype=np.float64).ravel()
    assert a.shape == o.shape == f.shape, (what, a.shape, o.shape, f.shape)
    assert np.isfinite(a).all(), f"{what}: non-finite outputs"
    ea, eo = np.abs(a - f), np.abs(o - f)
    stats = {"max_err": float(ea.max()), "mean_err": float(ea.mean()), "oracle_max_err": float(eo.max()),
             "oracle_mean_err": float(eo.mean()), "rms_f32": float(np.sqrt(np.mean(f ** 2)))}
    if not (ea.mean() <= mean_slack * eo.mean() and ea.max() <= max_slack * eo.max()):
        raise AssertionError(f"{what}: error vs float32 above the low-precision oracle's own (mean x{mean_slack}, "
                             f"max x{max_slack}): {stats}")
    return stats

"""Parity gates of the GPU attention tests.

Two bars, both asserted:
  * ELEMENT gate, the one the reference's own validator applies to its kernels
    (engine/src/gpu_attention_validation.rs:20-22, :378): for every element,
    |got - ref| <= 2e-5 + 2e-5 * |ref|, with ref the f64 oracle on the same inputs the kernel
    reads (fp16 pool values widened, the same query values). The kernels carry fp16 hi + lo
    halves of P and of an f32 query, so their error is far below it (about 1e-7 to 3e-6); a
    dropped lo half or a stale running max fails it. An fp16 output adds its own rounding,
    at most 2^-11 |ref| (round to nearest even).
  * NORTH-STAR bar, max-abs 2e-3 against the fp32 reference, checked on the
    same data; it is what the configuration tests on unrounded fp32 inputs assert, where the
    fp16 storage of K and V is part of the error.
"""
from __future__ import annotations

import numpy as np

ABS_TOL = 2e-5
REL_TOL = 2e-5
F16_REL = 2.0 ** -11
NORTH_STAR = 2e-3


def element_gate(got, want, what: str = "", out_f16: bool = False) -> float:
    """Assert the reference's element gate (plus fp16 output rounding when out_f16) and the
    north-star bar; return the max-abs error."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - want)
    bound = ABS_TOL + (REL_TOL + (F16_REL if out_f16 else 0.0)) * np.abs(want)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(int(np.argmax(err - bound)), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {err.size} elements outside |d| <= {ABS_TOL:g} + "
            f"{REL_TOL + (F16_REL if out_f16 else 0.0):g}|ref|; worst at {tuple(int(x) for x in i)}: "
            f"got {got[i]:.9e} ref {want[i]:.9e}")
    worst = float(err.max()) if err.size else 0.0
    assert worst <= NORTH_STAR, f"{what}: max-abs {worst:.3e} above {NORTH_STAR}"
    return worst


def north_star(got, want, what: str = "") -> float:
    """Max-abs error against the fp32 reference, asserted <= 2e-3; returned."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    worst = float(np.abs(got - want).max())
    assert worst <= NORTH_STAR, f"{what}: max-abs {worst:.3e} above {NORTH_STAR}"
    return worst

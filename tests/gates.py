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

The prefill kernels' default P16 precision carries P as one fp16 operand, rounded to nearest
even: each weight p_i moves by at most 2^-11 p_i, so an output moves by at most
2^-11 sum_i w_i |v_i| (w the row's softmax weights). Its element gate adds that term, with
vabs = the oracle's attention over |V| (attn_cases.oracle_abs_v): the bound the rounding
allows, on top of the reference's gate.
"""
from __future__ import annotations

import numpy as np

ABS_TOL = 2e-5
REL_TOL = 2e-5
F16_REL = 2.0 ** -11
P16_REL = 2.0 ** -11
NORTH_STAR = 2e-3


def element_gate(got, want, what: str = "", out_f16: bool = False, vabs=None) -> float:
    """Assert the reference's element gate (plus fp16 output rounding when out_f16, plus the
    P16 weight rounding 2^-11 * vabs when vabs is given) and the north-star bar; return the
    max-abs error."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - want)
    bound = ABS_TOL + (REL_TOL + (F16_REL if out_f16 else 0.0)) * np.abs(want)
    if vabs is not None:
        bound = bound + P16_REL * np.abs(np.asarray(vabs, np.float64))
    bad = err > bound
    if bad.any():
        i = np.unravel_index(int(np.argmax(err - bound)), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {err.size} elements outside |d| <= {ABS_TOL:g} + "
            f"{REL_TOL + (F16_REL if out_f16 else 0.0):g}|ref|"
            f"{' + 2^-11 sum w|v|' if vabs is not None else ''}; worst at "
            f"{tuple(int(x) for x in i)}: got {got[i]:.9e} ref {want[i]:.9e} "
            f"bound {bound[i]:.3e}")
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

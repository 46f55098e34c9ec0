"""The P16 element gate (gates.element_gate with vabs), pinned on the CPU.

The default prefill precision carries P as one fp16 operand rounded to nearest even, with l
summing the unrounded p. Each weight then moves by at most 2^-11 of itself, so an output
moves by at most 2^-11 sum_i w_i |v_i| from exact softmax weights; the gate adds that term
to the reference's element gate. Here numpy restates the P16 arithmetic (exact scores, p
rounded to fp16 RNE, f64 sums) on random and adversarial rows: it must pass the gate, and
the plausible mistakes it exists to catch must fail it: P truncated toward zero (the hi
half of the hi + lo pair used alone, on rows built so that the truncation errors add up),
a key dropped from a row, and a stale running max that lets P overflow fp16. The bound is
also reached within a small factor, so it is not loose by orders of magnitude.
"""
import numpy as np
import pytest

from gates import element_gate


def _rows(rng, n_rows, n_keys, d=64, q_scale=1.0):
    q = rng.standard_normal((n_rows, d)) * q_scale
    k = rng.standard_normal((n_keys, d))
    v = rng.standard_normal((n_keys, d))
    s = (q @ k.T) / np.sqrt(d)
    return s, v


def _exact(s, v):
    w = np.exp(s - s.max(axis=1, keepdims=True))
    w /= w.sum(axis=1, keepdims=True)
    return w @ v, w @ np.abs(v)


def _p16(s, v, rounding="rne", drop_key=None, stale_max=0.0):
    """P16 arithmetic: p = 2^(s log2e - m) (m the row max, or stale_max below it), p rounded
    to fp16 for the product, l = sum of the unrounded p (or of the rounded ones)."""
    m = s.max(axis=1, keepdims=True) - stale_max
    p = np.exp(s - m)
    if rounding == "rne":
        pr = p.astype(np.float16).astype(np.float64)
        l = p.sum(axis=1, keepdims=True)
    elif rounding == "rtz":
        bits = p.astype(np.float32).view(np.uint32) & np.uint32(0xFFFFE000)
        pr = bits.view(np.float32).astype(np.float64)
        l = p.sum(axis=1, keepdims=True)
    else:
        raise ValueError(rounding)
    if drop_key is not None:
        pr[:, drop_key] = 0.0
    return (pr @ v) / l


@pytest.mark.parametrize("q_scale", [0.25, 1.0, 4.0, 16.0])
@pytest.mark.parametrize("n_keys", [1, 2, 17, 64, 512])
def test_p16_arithmetic_passes_the_gate(q_scale, n_keys):
    rng = np.random.default_rng(1000 + n_keys + int(q_scale * 10))
    s, v = _rows(rng, 32, n_keys, q_scale=q_scale)
    want, vabs = _exact(s, v)
    got = _p16(s, v)
    element_gate(got, want, f"P16 n_keys {n_keys} q_scale {q_scale}", vabs=vabs)


def test_p16_bound_is_reached_within_a_factor_of_two():
    """Two keys of equal weight and far-apart values: the rounding error of the weights is
    as large as the bound allows up to a small factor, so the gate is not loose by orders of
    magnitude."""
    ratios = []
    for p1 in np.linspace(0.5, 1.0, 2001)[1:-1]:
        s = np.log(np.array([[1.0, p1]]))
        v = np.array([[4.0], [-4.0]])
        want, vabs = _exact(s, v)
        got = _p16(s, v)
        ratios.append(float(np.abs(got - want).max() / (2.0 ** -11 * vabs.max())))
    assert max(ratios) <= 1.0
    assert max(ratios) > 0.25


def test_truncated_p_fails_the_gate():
    """Weights whose p sits just above 0.5 lose almost 2^-10 of themselves to truncation
    (fp16 spacing 2^-11 in [0.5, 1)), against at most 2^-11 to rounding to nearest; with
    positive values the losses add up. One key at p = 1 sets the max."""
    n = 64
    s = np.full((1, n), np.log(0.5 + 0.999 * 2.0 ** -11))
    s[0, 0] = 0.0
    v = np.linspace(1.0, 2.0, n)[:, None] * np.ones((1, 8))
    want, vabs = _exact(s, v)
    element_gate(_p16(s, v), want, "P rounded to nearest", vabs=vabs)
    with pytest.raises(AssertionError):
        element_gate(_p16(s, v, rounding="rtz"), want, "P truncated", vabs=vabs)


def test_a_dropped_key_fails_the_gate():
    rng = np.random.default_rng(8)
    s, v = _rows(rng, 64, 96, q_scale=2.0)
    want, vabs = _exact(s, v)
    with pytest.raises(AssertionError):
        element_gate(_p16(s, v, drop_key=40), want, "key 40 dropped", vabs=vabs)


def test_p_overflowing_fp16_fails_the_gate():
    """A running max 20 (natural-log units) below the true one lets p reach e^20 > 65504:
    fp16 P overflows to inf and the output is not finite."""
    rng = np.random.default_rng(9)
    s, v = _rows(rng, 8, 64, q_scale=8.0)
    want, vabs = _exact(s, v)
    with np.errstate(over="ignore", invalid="ignore"):
        bad = _p16(s, v, stale_max=20.0)
    with pytest.raises(AssertionError):
        element_gate(bad, want, "stale max", vabs=vabs)

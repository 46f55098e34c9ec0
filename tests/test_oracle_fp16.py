"""Pins the oracle's fp16 conversion against numpy's IEEE binary16 (a library routine)."""
import numpy as np

import oracle


def test_f16_to_f32_matches_numpy_on_all_bit_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_bits_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_round_trips_every_finite_half():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = bits.view(np.float16).astype(np.float32)
    keep = ~np.isnan(vals)
    assert np.array_equal(oracle.f32_to_f16_bits(vals[keep]), bits[keep])


def test_f32_to_f16_rne_matches_numpy_on_random_and_edge_values():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200_000).astype(np.float32) * 4,
        rng.standard_normal(50_000).astype(np.float32) * 1e-5,    # subnormal halves
        rng.standard_normal(50_000).astype(np.float32) * 3e4,     # near overflow
        # exact midpoints between adjacent halves exercise ties-to-even
        ((np.arange(2048, dtype=np.float32) + 0.5) * 2.0 ** -10 + 1.0).astype(np.float32),
        np.array([0.0, -0.0, 65504, 65519.996, 65520, -65520, 1e-8, 2.0 ** -25,
                  2.0 ** -24, 3 * 2.0 ** -25, np.inf, -np.inf], np.float32),
    ])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_f16_bits(x), want)


def test_nan_stays_nan():
    h = oracle.f32_to_f16_bits(np.array([np.nan, -np.nan], np.float32))
    assert np.all(np.isnan(h.view(np.float16)))

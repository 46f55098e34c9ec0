"""The stamped diagnostic twin of the library and bench.py's phase summary (CPU only).

libcrucible_attn_stamps.so is the product library with the decode and prefill sources
compiled with -DCRUCIBLE_STAMPS: it must export everything the header declares plus the
stamp readers, and the product library must not export them. summarize_stamps turns stamp
rows into phase durations; here it runs on rows built by hand with known phase lengths.
"""
import ctypes
import os
import sys

import numpy as np
import pytest

from crucible_amd import _build, _lib

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402


def test_stamped_twin_exports_the_header_and_the_reader():
    if not os.path.exists(_build.STAMPS_LIB_PATH):
        pytest.skip("stamped library not built")
    twin = ctypes.CDLL(_build.STAMPS_LIB_PATH)
    for name in _lib.SIGNATURES:
        assert hasattr(twin, name), f"stamped library does not export {name}"
    for reader in ("crucible_debug_decode_stamps", "crucible_debug_prefill_stamps"):
        assert hasattr(twin, reader)
        assert not hasattr(_lib.load(), reader)


def _row(t0, phases, b, g, s, n_active, last):
    """Stamp slots from an entry time and phase lengths (ticks); slot 9 the meta word."""
    row = np.zeros(10, np.uint64)
    row[0] = t0
    t = t0
    for i, dt in enumerate(phases):
        t += dt
        row[i + 1] = t
    row[9] = (b | g << 16 | s << 24 | n_active << 32 | last << 48)
    return row


def test_summarize_stamps_recovers_known_phases():
    # unit (0, 0) in two splits, split 1 combines; unit (1, 0) in one split; one row of a
    # workgroup with no unit (kind 2) and one zero row, both ignored. Phases in order:
    # unit, issue, loads, compute, merge, publish, counter, combine.
    rows = np.zeros((16, 10), np.uint64)
    rows[0] = _row(1000, [20, 30, 100, 20, 30, 80, 40], 0, 0, 0, 2, 0)
    rows[1] = _row(1010, [25, 35, 90, 20, 40, 80, 50, 70], 0, 0, 1, 2, 1)
    rows[2] = _row(1005, [15, 25, 120, 10, 20, 60], 1, 0, 0, 1, 1)
    rows[2, 7:9] = 999_999  # an earlier launch's slots beyond a one-split unit's last
    rows[3, 0] = 1000
    rows[3, 9] = 2 << 52
    out = bench.summarize_stamps([rows], us_per_tick=0.01)
    ph = out["phases"]
    assert out["workgroups_per_launch"] == 3
    assert ph["skew"]["max_us"] == pytest.approx(0.10)
    assert ph["unit"]["median_us"] == pytest.approx(0.20)
    assert ph["issue"]["median_us"] == pytest.approx(0.30)
    assert ph["loads"]["max_us"] == pytest.approx(1.20)
    assert ph["counter"]["n"] == 2 and ph["counter"]["max_us"] == pytest.approx(0.50)
    assert ph["combine"]["n"] == 1 and ph["combine"]["median_us"] == pytest.approx(0.70)
    # the combining split ends last: 1010 + 410 ticks, 4.20 us after the first entry
    assert ph["chain"]["max_us"] == pytest.approx(4.20)
    crit = out["critical_workgroup"][0]
    assert crit["skew"] == pytest.approx(0.10) and crit["combine"] == pytest.approx(0.70)
    assert set(crit) == {"skew", *bench.PHASES}

"""Paging bookkeeping: the reference's own unit tests (C++ port) and the C API from Python."""
import os
import subprocess

import numpy as np
import pytest

from crucible_amd import _build
from crucible_amd._lib import CrucibleError
from crucible_amd.paged import PagePool, SequencePages, request_page_reservation, \
    segments_from_cu_seqlens


def test_reference_paging_kats_pass(tmp_path):
    """engine/src/paged.rs:244-496 and prefill.rs:394-453, ported to C++ (tests/paging_kat.cpp),
    built here with g++ against the library's host allocator source (no HIP)."""
    here = os.path.dirname(os.path.abspath(__file__))
    path = str(tmp_path / "paging_kat")
    subprocess.run([os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-Wall", "-Wextra",
                    "-I", _build.CSRC, os.path.join(here, "paging_kat.cpp"), os.path.join(_build.CSRC, "paging.cpp"),
                    "-o", path], check=True, capture_output=True, text=True)
    proc = subprocess.run([path], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "19 tests, 0 failed" in proc.stdout


def test_paging_kats_pass_under_address_and_undefined_sanitizers(tmp_path):
    """The same KATs with the allocator built under AddressSanitizer and UBSan (host code
    only, g++ on the CPU): every out-of-range id, double free and rollback path of
    paging.cpp runs with bounds, lifetime and overflow checks, and any report fails."""
    here = os.path.dirname(os.path.abspath(__file__))
    path = str(tmp_path / "paging_kat_san")
    subprocess.run([os.environ.get("CXX", "g++"), "-O1", "-g", "-std=c++17", "-Wall",
                    "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    "-fno-omit-frame-pointer", "-I", _build.CSRC,
                    os.path.join(here, "paging_kat.cpp"), os.path.join(_build.CSRC, "paging.cpp"),
                    "-o", path], check=True, capture_output=True, text=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    proc = subprocess.run([path], capture_output=True, text=True, timeout=120, env=env)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "19 tests, 0 failed" in proc.stdout
    assert "runtime error" not in proc.stderr and "AddressSanitizer" not in proc.stderr


def test_c_api_allocation_order_and_errors():
    pool = PagePool(4, 12, 192)
    assert [pool.alloc(), pool.alloc()] == [0, 1]
    pool.release(1)
    with pytest.raises(CrucibleError, match="double free"):
        pool.release(1)
    with pytest.raises(CrucibleError, match="out of range"):
        pool.release(7)


def test_c_api_sequence_growth_translation_and_rollback():
    pool = PagePool(3, 12, 192)
    s = SequencePages()
    s.grow(pool, 16 * 2 + 3)
    assert s.n_pages() == 3 and len(s) == 35
    pages = s.pages()
    assert s.translate(0) == (pages[0], 0)
    assert s.translate(17) == (pages[1], 1)
    with pytest.raises(CrucibleError):
        s.translate(35)
    t = s.table_padded(6)
    assert list(t[:3]) == list(pages) and list(t[3:]) == [0, 0, 0]
    s.release(pool)
    s.grow(pool, 16)
    with pytest.raises(CrucibleError, match="exhausted"):
        s.grow(pool, 16 * 4)
    assert pool.used_pages() == 1 and len(s) == 16


def test_reservation_and_segments_helpers():
    assert request_page_reservation(17, 17, 1024) == 3
    with pytest.raises(CrucibleError):
        request_page_reservation(1024, 2, 1024)
    seg, max_chunk = segments_from_cu_seqlens([0, 5, 5, 12], absolute_starts=[0, 3, 9])
    assert max_chunk == 7
    assert seg.tolist() == [[0, 5, 0, 0], [5, 0, 3, 1], [5, 7, 9, 2]]
    with pytest.raises(CrucibleError):
        segments_from_cu_seqlens([0, 5, 4])

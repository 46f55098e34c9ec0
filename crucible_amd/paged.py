"""Paged KV bookkeeping for Python callers, over the C++ restatement in the library.

``PagePool`` / ``SequencePages`` mirror engine/src/paged.rs:64-242 (stack free list,
first alloc is page 0, all-or-nothing growth, zero-padded tables) and
``request_page_reservation`` mirrors engine/src/prefill.rs:160-172. Errors raise
``CrucibleError`` with the reference's messages ("exhausted", "double free", ...).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import CrucibleError, PAGE_TOKENS


class PagePool:
    def __init__(self, n_pages: int, n_layer: int, kv_dim: int):
        self._lib = _lib.load()
        self._h = self._lib.crucible_page_pool_new(n_pages, n_layer, kv_dim)
        if not self._h:
            raise CrucibleError(*_lib.last_error())
        self.n_pages = n_pages

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._lib.crucible_page_pool_free(h)

    def free_pages(self) -> int:
        return self._lib.crucible_page_pool_free_pages(self._h)

    def used_pages(self) -> int:
        return self._lib.crucible_page_pool_used_pages(self._h)

    def alloc(self) -> int:
        page = self._lib.crucible_page_pool_alloc(self._h)
        if page < 0:
            raise CrucibleError(*_lib.last_error())
        return page

    def release(self, page: int) -> None:
        _lib.check(self._lib.crucible_page_pool_release(self._h, page))


class SequencePages:
    def __init__(self):
        self._lib = _lib.load()
        self._h = self._lib.crucible_seq_pages_new()

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._lib.crucible_seq_pages_free(h)

    def __len__(self) -> int:
        return self._lib.crucible_seq_pages_len(self._h)

    def n_pages(self) -> int:
        return self._lib.crucible_seq_pages_n_pages(self._h)

    def grow(self, pool: PagePool, extra: int) -> None:
        _lib.check(self._lib.crucible_seq_pages_grow(self._h, pool._h, extra))

    def release(self, pool: PagePool) -> None:
        _lib.check(self._lib.crucible_seq_pages_release(self._h, pool._h))

    def translate(self, pos: int) -> tuple[int, int]:
        page, slot = ctypes.c_int64(), ctypes.c_int64()
        _lib.check(self._lib.crucible_seq_pages_translate(self._h, pos, ctypes.byref(page),
                                                          ctypes.byref(slot)))
        return page.value, slot.value

    def table_padded(self, stride: int) -> np.ndarray:
        out = np.zeros(stride, np.int32)
        _lib.check(self._lib.crucible_seq_pages_table_padded(
            self._h, stride, out.ctypes.data_as(ctypes.c_void_p)))
        return out

    def pages(self) -> np.ndarray:
        return self.table_padded(self.n_pages())


def request_page_reservation(prompt: int, generated: int, context: int) -> int:
    pages = _lib.load().crucible_request_page_reservation(prompt, generated, context)
    if pages < 0:
        raise CrucibleError(*_lib.last_error())
    return pages


def segments_from_cu_seqlens(cu_seqlens, absolute_starts=None) -> tuple[np.ndarray, int]:
    """cu_seqlens[0..n] -> (segments int32[n, 4], max chunk length)."""
    cu = np.ascontiguousarray(cu_seqlens, np.int32)
    n = cu.size - 1
    starts = None if absolute_starts is None else np.ascontiguousarray(absolute_starts, np.int32)
    seg = np.zeros((n, 4), np.int32)
    max_chunk = _lib.load().crucible_segments_from_cu_seqlens(
        cu.ctypes.data_as(ctypes.c_void_p), n,
        None if starts is None else starts.ctypes.data_as(ctypes.c_void_p),
        seg.ctypes.data_as(ctypes.c_void_p))
    if max_chunk < 0:
        raise CrucibleError(*_lib.last_error())
    return seg, max_chunk


__all__ = ["PagePool", "SequencePages", "request_page_reservation", "segments_from_cu_seqlens",
           "PAGE_TOKENS"]

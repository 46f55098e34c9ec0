"""ctypes binding of ``libcrucible_attn.so`` (the C ABI in include/crucible_attn.h).

Loading fails loudly: there is no CPU fallback anywhere in the product path. Build the
library first (``__graft_entry__.build()`` or ``python -m crucible_amd._build``).
"""
from __future__ import annotations

import ctypes
import os

from . import _build

HEADER = os.path.join(os.path.dirname(_build.HERE), "include", "crucible_attn.h")

OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_WORKSPACE, ERR_LAUNCH = 0, 1, 2, 3, 4
F32, F16 = 0, 1
POOL_K, POOL_V = 0, 1
PARAM_SEQ, PARAM_PREFILL_POS = 3, 5
PAGE_TOKENS = 16
# launch-shape override keys (enum crucible_tuning_key) and the decode order values
TUNE_KEYS = {"decode_pages": 0, "decode_waves": 1, "decode_order": 2, "prefill_direct": 3,
             "prefill_heavy_first": 4, "prefill_qb": 5, "prefill_bufs": 6, "linear_tile": 7,
             "decode_combine_width": 8, "prefill_p16": 9,
             "prefill_m32": 10, "prefill_persist": 11, "linear_prefetch": 12}
DECODE_ORDERS = {"split": 0, "request": 1, "compact": 2}

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t

# name -> (argtypes, restype); every symbol declared in the header.
SIGNATURES = {
    "crucible_attn_version": ([], ctypes.c_char_p),
    "crucible_attn_last_error": ([ctypes.c_char_p, _SZ], _I),
    "crucible_attn_set_tuning": ([_I, _I], _I),
    "crucible_attn_get_tuning": ([_I], _I),
    "crucible_attn_tuning_name": ([_I], ctypes.c_char_p),
    "crucible_cache_store": ([_P, _I, _P, _I, _I64, _I64, _I64, _I64, _P], _I),
    "crucible_cache_store_paged": ([_P, _I, _P, _I, _P, _I64, _I64, _I64, _I64, _P, _P], _I),
    "crucible_cache_store_rows_paged": ([_P, _I, _P, _I, _P, _P, _I64, _I64, _I64, _I64, _I64, _P], _I),
    "crucible_cache_store_packed_paged": ([_P, _I, _P, _I, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P], _I),
    "crucible_attention_decode_workspace_bytes": ([_I64, _I64, _I64], _SZ),
    "crucible_attention_decode_paged": ([_P, _I, _P, _P, _P, _I, _P, _P] + [_I64] * 9 + [_P, _SZ, _P], _I),
    "crucible_attention_decode_paged_append": ([_P, _I, _P, _P, _I, _P, _P, _P, _I, _P, _P, _P] + [_I64] * 9 + [_P, _SZ, _P], _I),
    "crucible_attention_decode_paged_append_noalloc": ([_P, _I, _P, _P, _I, _P, _P, _P, _I, _P, _P, _P] + [_I64] * 9 + [_P], _I),
    "crucible_attention_decode_kernel_name": ([_I64, _I64, _I64, _I64, _I, _I, ctypes.c_char_p, _SZ], _I),
    "crucible_attention_decode_qkv_paged_append": ([_P, _I64, _P, _P, _I64, _P, _P, _P, _I, _P, _P, _P] + [_I64] * 9 + [_P, _SZ, _P], _I),
    "crucible_attention_decode": ([_P, _I, _P, _P, _P, _I, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P, _SZ, _P], _I),
    "crucible_attention_split": ([_P, _I, _P, _P, _P, _P, _P, _P, _I, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P], _I),
    "crucible_attention_prefill_paged": ([_P, _I, _P, _P, _P, _I, _P] + [_I64] * 8 + [_P, _P], _I),
    "crucible_attention_prefill_packed": ([_P, _I, _P, _P, _P, _I, _P, _P, _P] + [_I64] * 9 + [_P], _I),
    "crucible_attention_prefill_tiled": ([_P, _I, _P, _P, _P, _P, _P, _I, _P, _P] + [_I64] * 9 + [_I, _I64, _P], _I),
    "crucible_attention_prefill": ([_P, _I, _P, _P, _P, _I] + [_I64] * 8 + [_P], _I),
    "crucible_argmax_rows": ([_P, _P, _I64, _I64, _P], _I),
    "crucible_greedy_advance": ([_P, _I64, _I64, _P, _I64, _P, _I64, _P, _P, _P, _I64, _P, _P,
                                 _P, _P], _I),
    "crucible_linear_f64acc": ([_P, _I64, _P, ctypes.c_float, _P, _I64, _I64, _P, _P, _I64, _I64,
                                _P], _I),
    "crucible_linear_swiglu_f64acc": ([_P, _I64, _P, ctypes.c_float, _P, _P, _I64, _I64, _P,
                                       _I64, _I64, _P], _I),
    "crucible_linear_f64acc_prefetch": ([_P, _I64, _P, ctypes.c_float, _P, _I64, _I64, _P, _P,
                                         _I64, _I64, _P, _I64, _P], _I),
    "crucible_linear_swiglu_f64acc_prefetch": ([_P, _I64, _P, ctypes.c_float, _P, _P, _I64,
                                                _I64, _P, _I64, _I64, _P, _I64, _P], _I),
    "crucible_rmsnorm_rows": ([_P, _I64, _P, ctypes.c_float, _P, _I64, _I64, _I64, _P], _I),
    "crucible_rope_split_qkv": ([_P, _I64, _P, _P, _P, _P, _P, _P] + [_I64] * 5 + [_P], _I),
    "crucible_segments_from_cu_seqlens": ([_P, _I64, _P, _P], _I64),
    "crucible_page_pool_new": ([_I64, _I64, _I64], _P),
    "crucible_page_pool_free": ([_P], None),
    "crucible_page_pool_free_pages": ([_P], _I64),
    "crucible_page_pool_used_pages": ([_P], _I64),
    "crucible_page_pool_alloc": ([_P], _I64),
    "crucible_page_pool_release": ([_P, _I64], _I),
    "crucible_seq_pages_new": ([], _P),
    "crucible_seq_pages_free": ([_P], None),
    "crucible_seq_pages_len": ([_P], _I64),
    "crucible_seq_pages_n_pages": ([_P], _I64),
    "crucible_seq_pages_grow": ([_P, _P, _I64], _I),
    "crucible_seq_pages_release": ([_P, _P], _I),
    "crucible_seq_pages_translate": ([_P, _I64, _P, _P], _I),
    "crucible_seq_pages_table_padded": ([_P, _I64, _P], _I),
    "crucible_request_page_reservation": ([_I64, _I64, _I64], _I64),
}


class CrucibleError(RuntimeError):
    """A non-zero status from the C ABI, with the library's message."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[status {status}] {message}")
        self.status = status


_lib = None


def load(path: str | None = None):
    """Load and bind the shared library (once)."""
    global _lib
    if _lib is not None:
        return _lib
    path = path or _build.LIB_PATH
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build it with __graft_entry__.build() or "
            "`python -m crucible_amd._build` (hipcc, gfx950). There is no CPU fallback.")
    lib = ctypes.CDLL(path)
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def last_error() -> tuple[int, str]:
    buf = ctypes.create_string_buffer(512)
    status = load().crucible_attn_last_error(buf, len(buf))
    return status, buf.value.decode(errors="replace")


def check(status: int) -> None:
    if status != OK:
        _, msg = last_error()
        raise CrucibleError(status, msg)

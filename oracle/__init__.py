"""CPU oracle for the crucible attention hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker. The product
(``crucible_amd``) never imports it; the product fails loudly when its HIP
library is missing instead of falling back to anything here.

This module is a thin numpy/ctypes wrapper over ``oracle/oracle.c``, which
restates the reference arithmetic (citations are in that file's header and on
each function below). ``build()`` compiles it with gcc.

Parity pins (tests that check the oracle itself, not the GPU):
  tests/test_oracle_fp16.py      f32<->f16 vs numpy float16
  tests/test_oracle_paging.py    geometry KATs, append/gather round trips
  tests/test_oracle_attention.py torch SDPA, numpy textbook, closed forms,
                                 f64 vs reference-order f32, split/combine algebra
  tests/test_oracle_misc.py      argmax adversarial rows, RoPE KATs, generators
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

PAGE_TOKENS = 16
STORE_ROWS, STORE_PARAMS, STORE_PACKED, STORE_CONTIG = 0, 1, 2, 3
POOL_K, POOL_V = 0, 1


def build() -> str:
    """Compile oracle.c into oracle/_build/liboracle.so (gcc)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    """The built oracle library. It is never built here: a test process may already hold
    the GPU, and starting ``make`` from it would fork a GPU-initialised process. Build it
    beforehand (``oracle.build()``, ``__graft_entry__.build()``)."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH}; build it first "
                               "(python -c 'import oracle; oracle.build()', or "
                               "__graft_entry__.build())")
        _lib = _bind(ctypes.CDLL(_LIB_PATH))
    return _lib


def _bind(L):
    P = ctypes.c_void_p
    I64 = ctypes.c_int64
    U64 = ctypes.c_uint64
    D = ctypes.c_double
    I = ctypes.c_int
    sig = {
        "orc_f32_to_f16": ([ctypes.c_float], ctypes.c_uint16),
        "orc_f16_to_f32": ([ctypes.c_uint16], ctypes.c_float),
        "orc_f32_to_f16_array": ([P, P, I64], None),
        "orc_f16_to_f32_array": ([P, P, I64], None),
        "orc_paged_offset": ([I64] * 5, I64),
        "orc_pool_index": ([I] + [I64] * 6, I64),
        "orc_contig_index": ([I, I64, I64, I64, I64], I64),
        "orc_cache_store": ([I, I, P, P, P, P, P, P, P] + [I64] * 7, None),
        "orc_gather": ([I, P, P, I64, I64, I64, I64, P], None),
        "orc_v_blocks_transpose": ([P, P, I64, I64, I], None),
        "orc_attention_dense": ([P, P, P, P, I64, I64, I64, I64, I64, D, I, P], I),
        "orc_attention_paged_rows": ([P, P, P, P, P, P] + [I64] * 7 + [D, I, P], I),
        "orc_split_partials": ([P, P, P, I64, I64, I64, D, I64, I64, P, P, P], None),
        "orc_split_combine": ([P, P, P, I64, I64, P], None),
        "orc_argmax": ([P, I64], I64),
        "orc_rope_table": ([I64, I64, D, P, P], None),
        "orc_rope_apply": ([P, I64, P, P, I64], None),
        "orc_xorshift": ([P], U64),
        "orc_probe_tokens": ([I64, I64, P], None),
        "orc_shuffle": ([U64, I64, P], None),
        "orc_value": ([U64] * 5, ctypes.c_float),
        "orc_splitmix64": ([P], U64),
        "orc_normal_f32": ([U64, I64, I64, P], None),
        "orc_normal_f16": ([U64, I64, I64, P], None),
        "orc_value_grid": ([U64, I64, I64, I64, I64, U64, P], None),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    return L


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- fp16

def f32_to_f16_bits(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


# ---------------------------------------------------------------- geometry / append

def paged_offset(page, slot, n_layer, layer, kv_dim) -> int:
    return lib().orc_paged_offset(page, slot, n_layer, layer, kv_dim)


def pool_index(kind, page, slot, c, n_layer, layer, kv_dim) -> int:
    return lib().orc_pool_index(kind, page, slot, c, n_layer, layer, kv_dim)


def cache_store(mode, kind, pool, src, *, tables=None, positions=None, owners=None,
                params=None, rows, kv_dim, table_stride=0, n_layer=1, layer=0,
                layer_base=0, pos_offset=0):
    """Scatter rows into ``pool`` (uint16 fp16 bits, modified in place).

    ``src`` float32 rows are rounded to fp16 (RNE); uint16 rows are copied.
    """
    assert pool.dtype == np.uint16 and pool.flags.c_contiguous
    src_f32 = src_f16 = None
    if src.dtype == np.uint16:
        src_f16 = _c(src, np.uint16)
    else:
        src_f32 = _c(src, np.float32)
    lib().orc_cache_store(mode, kind, _p(src_f32), _p(src_f16), _p(pool),
                          _p(_c(tables, np.int32)), _p(_c(positions, np.int32)),
                          _p(_c(owners, np.int32)), _p(_c(params, np.int32)),
                          rows, kv_dim, table_stride, n_layer, layer, layer_base, pos_offset)


def gather(kind, pool, table, length, kv_dim, n_layer, layer) -> np.ndarray:
    out = np.empty((length, kv_dim), np.float32)
    lib().orc_gather(kind, _p(_c(pool, np.uint16)), _p(_c(table, np.int32)), length, kv_dim,
                     n_layer, layer, _p(out))
    return out


def v_blocks_to_reference(v_pool, kv_dim) -> np.ndarray:
    v = _c(v_pool, np.uint16)
    out = np.empty_like(v)
    lib().orc_v_blocks_transpose(_p(v), _p(out), v.size // (PAGE_TOKENS * kv_dim), kv_dim, 1)
    return out


def v_blocks_from_reference(v_ref, kv_dim) -> np.ndarray:
    v = _c(v_ref, np.uint16)
    out = np.empty_like(v)
    lib().orc_v_blocks_transpose(_p(v), _p(out), v.size // (PAGE_TOKENS * kv_dim), kv_dim, 0)
    return out


# ---------------------------------------------------------------- attention

def attention_dense(q, k, v, lens, n_head, n_kv_head, head_dim, scale=None, precise=True):
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    v = _c(v, np.float32)
    lens = _c(lens, np.int32)
    n_q = lens.size
    n_k = k.shape[0]
    out = np.zeros((n_q, n_head * head_dim), np.float32)
    scale = 1.0 / np.sqrt(head_dim) if scale is None else scale
    rc = lib().orc_attention_dense(_p(q), _p(k), _p(v), _p(lens), n_q, n_k, n_head, n_kv_head,
                                   head_dim, float(scale), int(precise), _p(out))
    if rc:
        raise ValueError(f"orc_attention_dense failed ({rc})")
    return out


def attention_paged_rows(q, k_pool, v_pool, tables, lens, *, table_index=None, n_head,
                         n_kv_head, head_dim, table_stride, n_layer, layer, scale=None,
                         precise=True, out=None):
    """One query row per entry; row r sees keys [0, lens[r]) through its table."""
    q = _c(q, np.float32)
    lens = _c(lens, np.int32)
    rows = lens.size
    if out is None:
        out = np.zeros((rows, n_head * head_dim), np.float32)
    scale = 1.0 / np.sqrt(head_dim) if scale is None else scale
    rc = lib().orc_attention_paged_rows(
        _p(q), _p(_c(k_pool, np.uint16)), _p(_c(v_pool, np.uint16)), _p(_c(tables, np.int32)),
        _p(_c(table_index, np.int32)), _p(lens), rows, n_head, n_kv_head, head_dim,
        table_stride, n_layer, layer, float(scale), int(precise), _p(out))
    if rc:
        raise ValueError(f"orc_attention_paged_rows failed ({rc})")
    return out


def split_partials(q, k, v, length, head_dim, chunk, n_chunks, scale=None, stride=None):
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    v = _c(v, np.float32)
    stride = head_dim if stride is None else stride
    pm = np.empty(n_chunks, np.float64)
    pl = np.empty(n_chunks, np.float64)
    po = np.empty((n_chunks, head_dim), np.float64)
    scale = 1.0 / np.sqrt(head_dim) if scale is None else scale
    lib().orc_split_partials(_p(q), _p(k), _p(v), length, stride, head_dim, float(scale),
                             chunk, n_chunks, _p(pm), _p(pl), _p(po))
    return pm, pl, po


def split_combine(pm, pl, po):
    pm = _c(pm, np.float64)
    pl = _c(pl, np.float64)
    po = _c(po, np.float64)
    out = np.empty(po.shape[1], np.float64)
    lib().orc_split_combine(_p(pm), _p(pl), _p(po), pm.size, po.shape[1], _p(out))
    return out


# ---------------------------------------------------------------- selection / rope

def argmax(row) -> int:
    row = _c(row, np.float32)
    return int(lib().orc_argmax(_p(row), row.size))


def rope_table(head_dim, max_seq, theta=10000.0):
    half = head_dim // 2
    cos_t = np.empty((max_seq, half), np.float32)
    sin_t = np.empty((max_seq, half), np.float32)
    lib().orc_rope_table(head_dim, max_seq, float(theta), _p(cos_t), _p(sin_t))
    return cos_t, sin_t


def rope_apply(vec, cos_t, sin_t, pos):
    vec = np.array(vec, np.float32, copy=True)
    lib().orc_rope_apply(_p(vec), vec.size, _p(_c(cos_t, np.float32)),
                         _p(_c(sin_t, np.float32)), pos)
    return vec


# ---------------------------------------------------------------- generators

def xorshift_stream(state: int, n: int) -> list[int]:
    st = ctypes.c_uint64(state)
    return [lib().orc_xorshift(ctypes.byref(st)) for _ in range(n)]


def probe_tokens(n, vocab) -> np.ndarray:
    out = np.empty(n, np.int64)
    lib().orc_probe_tokens(n, vocab, _p(out))
    return out


def shuffle(seed, n) -> np.ndarray:
    out = np.empty(n, np.int64)
    lib().orc_shuffle(seed, n, _p(out))
    return out


def value(id_, pos, head, dim, salt) -> float:
    return float(lib().orc_value(id_, pos, head, dim, salt))


def value_grid(id_, pos0, n_pos, n_head, head_dim, salt) -> np.ndarray:
    out = np.empty((n_pos, n_head, head_dim), np.float32)
    lib().orc_value_grid(id_, pos0, n_pos, n_head, head_dim, salt, _p(out))
    return out


def splitmix64_stream(state: int, n: int) -> list[int]:
    st = ctypes.c_uint64(state)
    return [lib().orc_splitmix64(ctypes.byref(st)) for _ in range(n)]


def normal_f32(seed, n, start=0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_normal_f32(seed, start, n, _p(out))
    return out


def normal_f16(seed, n, start=0) -> np.ndarray:
    out = np.empty(n, np.uint16)
    lib().orc_normal_f16(seed, start, n, _p(out))
    return out

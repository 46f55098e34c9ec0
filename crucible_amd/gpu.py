"""Host-side mirror of the reference engine's attention launch API.

``Gpu`` has the attention and KV-append methods of ``impl Gpu`` in the reference
(engine/src/gpu.rs), with the same names, argument order and meaning, over torch
device tensors. Each method checks its tensors (device, dtype, contiguity, capacity,
as the reference checks slice lengths), calls the C ABI, and raises ``CrucibleError``
on any non-zero status. Everything runs on the caller's current HIP stream, nothing
synchronises, and nothing here computes attention itself: the HIP library is the only
implementation and loading fails if it is missing.

Differences from the reference, all from the allowed page-layout change:
  * pools are fp16 (reference: f32) and V pools store each (page, layer) block
    transposed, so the append methods take ``kind="k"`` or ``kind="v"``;
  * split-K decode needs a workspace; pass one (graph capture) or let the Gpu keep
    a cached one per (batch, n_head, max_seq).
"""
from __future__ import annotations

import contextlib

import torch

from . import _lib
from ._lib import CrucibleError, F16, F32, POOL_K, POOL_V, PAGE_TOKENS

_DTYPES = {torch.float32: F32, torch.float16: F16}
_KINDS = {"k": POOL_K, "v": POOL_V, POOL_K: POOL_K, POOL_V: POOL_V}


def _ptr(t):
    return None if t is None else ctypes_ptr(t)


def ctypes_ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def _dtype(t: torch.Tensor, what: str) -> int:
    if t.dtype not in _DTYPES:
        raise CrucibleError(_lib.ERR_INVALID, f"{what}: dtype {t.dtype} (need float32/float16)")
    return _DTYPES[t.dtype]


def _need(t, what, *, dtype=None, numel=None):
    if t is None:
        raise CrucibleError(_lib.ERR_INVALID, f"{what} is required")
    if not t.is_cuda:
        raise CrucibleError(_lib.ERR_INVALID, f"{what} must be a device tensor")
    if not t.is_contiguous():
        raise CrucibleError(_lib.ERR_INVALID, f"{what} must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise CrucibleError(_lib.ERR_INVALID, f"{what}: dtype {t.dtype}, expected {dtype}")
    if numel is not None and t.numel() < numel:
        raise CrucibleError(_lib.ERR_INVALID, f"{what}: {t.numel()} elements, need {numel}")
    return t


def _prefetch_region(t):
    """(pointer, bytes) of a prefetch tensor: contiguous on the device, whole 64-byte lines
    (a trailing partial line is left out)."""
    _need(t, "prefetch")
    return _ptr(t), (t.numel() * t.element_size()) // 64 * 64


def set_tuning(**overrides) -> None:
    """Force launch shapes for every later launch in the process (crucible_attn_set_tuning):
    decode_pages, decode_waves, decode_order ("split" | "request" | "compact"),
    prefill_direct, prefill_heavy_first, prefill_qb, prefill_bufs, linear_tile,
    decode_combine_width, prefill_p16, prefill_m32, prefill_persist, linear_prefetch. None
    returns a key to the launcher's own choice."""
    lib = _lib.load()
    for name, value in overrides.items():
        if name not in _lib.TUNE_KEYS:
            raise CrucibleError(_lib.ERR_INVALID, f"unknown tuning key {name!r}")
        if value is None:
            v = -1
        elif name == "decode_order" and isinstance(value, str):
            v = _lib.DECODE_ORDERS[value]
        else:
            v = int(value)
        _lib.check(lib.crucible_attn_set_tuning(_lib.TUNE_KEYS[name], v))


def tuning_state() -> dict:
    """The overrides in force, by environment-variable name (automatic keys left out)."""
    lib = _lib.load()
    out = {}
    for key in _lib.TUNE_KEYS.values():
        v = lib.crucible_attn_get_tuning(key)
        if v != -1:
            out[lib.crucible_attn_tuning_name(key).decode()] = v
    return out


@contextlib.contextmanager
def tuning(**overrides):
    """set_tuning for the duration of a with-block; the previous values come back after."""
    lib = _lib.load()
    saved = {name: lib.crucible_attn_get_tuning(key) for name, key in _lib.TUNE_KEYS.items()
             if name in overrides}
    try:
        set_tuning(**overrides)
        yield
    finally:
        for name, v in saved.items():
            _lib.check(lib.crucible_attn_set_tuning(_lib.TUNE_KEYS[name], v))


def pool_elems(n_pages: int, n_layer: int, kv_dim: int) -> int:
    """Elements of one fp16 pool: [n_pages][n_layer][16][kv_dim] (paged.rs:14-21)."""
    return n_pages * n_layer * PAGE_TOKENS * kv_dim


class Gpu:
    """The attention/append subset of the reference ``Gpu`` (engine/src/gpu.rs:327-2157)."""

    def __init__(self, device: int | torch.device = 0):
        self.lib = _lib.load()
        self.device = torch.device("cuda", device) if isinstance(device, int) else device
        self._workspaces: dict[tuple, torch.Tensor] = {}
        self._bindings: dict[tuple, tuple] = {}  # workspace key -> pools it last served

    # ------------------------------------------------------------- plumbing
    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def workspace(self, batch: int, n_head: int, max_seq: int, pools=None) -> torch.Tensor:
        """Split-K scratch for decode, allocated once per shape (never inside a call).

        ``pools`` is the call's ``(k_pool, v_pool)``. The workspace's unit plan holds page
        ids read for one table and pair of pools, and the kernel takes an entry only for the
        same three addresses; a pool freed and allocated again at the same address with
        fewer pages would pass that check. So the cached workspace remembers the pools'
        addresses and sizes and is zeroed (on the current stream, ordered before the call)
        whenever they change."""
        key = (batch, n_head, max_seq)
        ws = self._workspaces.get(key)
        if ws is None:
            nbytes = self.lib.crucible_attention_decode_workspace_bytes(batch, n_head, max_seq)
            ws = torch.zeros(max(nbytes, 16), dtype=torch.uint8, device=self.device)
            self._workspaces[key] = ws
        if pools is not None:
            binding = tuple((t.data_ptr(), t.numel()) for t in pools)
            if self._bindings.get(key, binding) != binding:
                ws.zero_()
            self._bindings[key] = binding
        return ws

    @staticmethod
    def version() -> str:
        return _lib.load().crucible_attn_version().decode()

    # ------------------------------------------------------------- KV append
    def cache_store(self, src, cache, rows, kv_dim, layer_base, pos_offset, *, kind):
        """gpu.rs:1259-1279: contiguous cache, position pos_offset + row."""
        _need(src, "src", numel=rows * kv_dim)
        _need(cache, "cache", dtype=torch.float16)
        _lib.check(self.lib.crucible_cache_store(
            _ptr(src), _dtype(src, "src"), _ptr(cache), _KINDS[kind], rows, kv_dim, layer_base,
            pos_offset, self._stream()))

    def cache_store_paged(self, src, pool, page_table, rows, kv_dim, n_layer, layer, params, *,
                          kind):
        """gpu.rs:1281-1307: one table, position params[5] + row."""
        _need(src, "src", numel=rows * kv_dim)
        _need(pool, "pool", dtype=torch.float16)
        _need(page_table, "page_table", dtype=torch.int32)
        _need(params, "params", dtype=torch.int32, numel=6)
        _lib.check(self.lib.crucible_cache_store_paged(
            _ptr(src), _dtype(src, "src"), _ptr(pool), _KINDS[kind], _ptr(page_table), rows,
            kv_dim, n_layer, layer, _ptr(params), self._stream()))

    def cache_store_rows_paged(self, src, pool, page_tables, positions, rows, kv_dim,
                               table_stride, n_layer, layer, *, kind):
        """gpu.rs:1405-1439: row r at positions[r] through its own table row."""
        _need(src, "src", numel=rows * kv_dim)
        _need(pool, "pool", dtype=torch.float16)
        _need(page_tables, "page_tables", dtype=torch.int32, numel=rows * table_stride)
        _need(positions, "positions", dtype=torch.int32, numel=rows)
        _lib.check(self.lib.crucible_cache_store_rows_paged(
            _ptr(src), _dtype(src, "src"), _ptr(pool), _KINDS[kind], _ptr(page_tables),
            _ptr(positions), rows, kv_dim, table_stride, n_layer, layer, self._stream()))

    def cache_store_packed_paged(self, src, pool, tables, owners, positions, rows, kv_dim,
                                 table_stride, n_layer, layer, *, kind):
        """gpu.rs:1800-1835: row r at positions[r] through tables[owners[r]]."""
        _need(src, "src", numel=rows * kv_dim)
        _need(pool, "pool", dtype=torch.float16)
        _need(tables, "tables", dtype=torch.int32)
        _need(owners, "owners", dtype=torch.int32, numel=rows)
        _need(positions, "positions", dtype=torch.int32, numel=rows)
        _lib.check(self.lib.crucible_cache_store_packed_paged(
            _ptr(src), _dtype(src, "src"), _ptr(pool), _KINDS[kind], _ptr(tables), _ptr(owners),
            _ptr(positions), rows, kv_dim, table_stride, n_layer, layer, self._stream()))

    # ------------------------------------------------------------- decode
    def attention_decode_paged(self, q, k_pool, v_pool, out, page_tables, seq_lens, batch,
                               n_head, n_kv_head, head_dim, table_stride, n_layer, layer,
                               kv_dim, max_seq, workspace=None):
        """gpu.rs:1441-1500. seq_lens[b] <= 0: request b inactive, out untouched."""
        _need(q, "q", numel=batch * n_head * head_dim)
        _need(out, "out", numel=batch * n_head * head_dim)
        _need(k_pool, "k_pool", dtype=torch.float16)
        _need(v_pool, "v_pool", dtype=torch.float16)
        _need(page_tables, "page_tables", dtype=torch.int32, numel=batch * table_stride)
        _need(seq_lens, "seq_lens", dtype=torch.int32, numel=batch)
        ws = workspace if workspace is not None else self.workspace(batch, n_head, max_seq,
                                                                   (k_pool, v_pool))
        _need(ws, "workspace")
        _lib.check(self.lib.crucible_attention_decode_paged(
            _ptr(q), _dtype(q, "q"), _ptr(k_pool), _ptr(v_pool), _ptr(out), _dtype(out, "out"),
            _ptr(page_tables), _ptr(seq_lens), batch, n_head, n_kv_head, head_dim, table_stride,
            n_layer, layer, kv_dim, max_seq, _ptr(ws), ws.numel() * ws.element_size(),
            self._stream()))

    def attention_decode_paged_append(self, q, k_new, v_new, k_pool, v_pool, out, page_tables,
                                      positions, seq_lens, batch, n_head, n_kv_head, head_dim,
                                      table_stride, n_layer, layer, kv_dim, max_seq,
                                      workspace=None):
        """Fused gpu_model.rs:1434-1507 sequence: append K and V rows at positions[b], then
        decode with seq_lens, in one launch (same pool bytes and output as the three calls)."""
        _need(q, "q", numel=batch * n_head * head_dim)
        _need(out, "out", numel=batch * n_head * head_dim)
        _need(k_new, "k_new", numel=batch * kv_dim)
        _need(v_new, "v_new", dtype=k_new.dtype, numel=batch * kv_dim)
        _need(k_pool, "k_pool", dtype=torch.float16)
        _need(v_pool, "v_pool", dtype=torch.float16)
        _need(page_tables, "page_tables", dtype=torch.int32, numel=batch * table_stride)
        _need(positions, "positions", dtype=torch.int32, numel=batch)
        _need(seq_lens, "seq_lens", dtype=torch.int32, numel=batch)
        ws = workspace if workspace is not None else self.workspace(batch, n_head, max_seq,
                                                                   (k_pool, v_pool))
        _lib.check(self.lib.crucible_attention_decode_paged_append(
            _ptr(q), _dtype(q, "q"), _ptr(k_new), _ptr(v_new), _dtype(k_new, "k_new"),
            _ptr(k_pool), _ptr(v_pool), _ptr(out), _dtype(out, "out"), _ptr(page_tables),
            _ptr(positions), _ptr(seq_lens), batch, n_head, n_kv_head, head_dim, table_stride,
            n_layer, layer, kv_dim, max_seq, _ptr(ws), ws.numel() * ws.element_size(),
            self._stream()))

    def attention_decode_qkv_paged_append(self, qkv, rope_cos, rope_sin, k_pool, v_pool, out,
                                          page_tables, positions, seq_lens, batch, n_head,
                                          n_kv_head, head_dim, table_stride, n_layer, layer,
                                          kv_dim, max_seq, workspace=None):
        """The fused step fed from the fused q/k/v rows, with RoPE of q and k at positions[b]
        (rope tables [max_pos][head_dim/2] f32, or None for no rotation)."""
        _need(qkv, "qkv", dtype=torch.float32)
        row_stride = qkv.shape[1]
        _need(qkv, "qkv", numel=batch * row_stride)
        _need(out, "out", numel=batch * n_head * head_dim)
        _need(k_pool, "k_pool", dtype=torch.float16)
        _need(v_pool, "v_pool", dtype=torch.float16)
        _need(page_tables, "page_tables", dtype=torch.int32, numel=batch * table_stride)
        _need(positions, "positions", dtype=torch.int32, numel=batch)
        _need(seq_lens, "seq_lens", dtype=torch.int32, numel=batch)
        max_pos = 0
        if rope_cos is not None:
            _need(rope_cos, "rope_cos", dtype=torch.float32)
            _need(rope_sin, "rope_sin", dtype=torch.float32, numel=rope_cos.numel())
            max_pos = rope_cos.shape[0]
        ws = workspace if workspace is not None else self.workspace(batch, n_head, max_seq,
                                                                   (k_pool, v_pool))
        _lib.check(self.lib.crucible_attention_decode_qkv_paged_append(
            _ptr(qkv), row_stride, _ptr(rope_cos), _ptr(rope_sin), max_pos, _ptr(k_pool),
            _ptr(v_pool), _ptr(out), _dtype(out, "out"), _ptr(page_tables), _ptr(positions),
            _ptr(seq_lens), batch, n_head, n_kv_head, head_dim, table_stride, n_layer, layer,
            kv_dim, max_seq, _ptr(ws), ws.numel() * ws.element_size(), self._stream()))

    def attention_decode(self, q, k_cache, v_cache, out, n_head, n_kv_head, head_dim, params,
                         max_seq, cache_stride, layer_base, workspace=None):
        """gpu.rs:762-817: contiguous cache, length params[3]."""
        _need(q, "q", numel=n_head * head_dim)
        _need(out, "out", numel=n_head * head_dim)
        _need(k_cache, "k_cache", dtype=torch.float16)
        _need(v_cache, "v_cache", dtype=torch.float16)
        _need(params, "params", dtype=torch.int32, numel=6)
        ws = workspace if workspace is not None else self.workspace(1, n_head, max_seq)
        _lib.check(self.lib.crucible_attention_decode(
            _ptr(q), _dtype(q, "q"), _ptr(k_cache), _ptr(v_cache), _ptr(out), _dtype(out, "out"),
            n_head, n_kv_head, head_dim, _ptr(params), max_seq, cache_stride, layer_base,
            _ptr(ws), ws.numel() * ws.element_size(), self._stream()))

    def attention_split(self, q, k_cache, v_cache, partial_o, partial_m, partial_l, out, n_head,
                        n_kv_head, head_dim, params, capacity, cache_stride, layer_base):
        """gpu.rs:1936-2014: flash-decoding with caller-owned partials (128-token chunks)."""
        n_chunks = -(-capacity // 128)
        _need(q, "q", numel=n_head * head_dim)
        _need(out, "out", numel=n_head * head_dim)
        _need(partial_o, "partial_o", dtype=torch.float32, numel=n_head * n_chunks * head_dim)
        _need(partial_m, "partial_m", dtype=torch.float32, numel=n_head * n_chunks)
        _need(partial_l, "partial_l", dtype=torch.float32, numel=n_head * n_chunks)
        _need(params, "params", dtype=torch.int32, numel=6)
        _lib.check(self.lib.crucible_attention_split(
            _ptr(q), _dtype(q, "q"), _ptr(k_cache), _ptr(v_cache), _ptr(partial_o),
            _ptr(partial_m), _ptr(partial_l), _ptr(out), _dtype(out, "out"), n_head, n_kv_head,
            head_dim, _ptr(params), capacity, cache_stride, layer_base, self._stream()))

    # ------------------------------------------------------------- prefill
    def attention_prefill_paged(self, q, k_pool, v_pool, out, page_table, rows, n_head,
                                n_kv_head, head_dim, n_layer, layer, kv_dim, max_seq, params):
        """gpu.rs:1502-1549: one sequence, row r at position params[5] + r."""
        _need(q, "q", numel=rows * n_head * head_dim)
        _need(out, "out", numel=rows * n_head * head_dim)
        _need(page_table, "page_table", dtype=torch.int32)
        _need(params, "params", dtype=torch.int32, numel=6)
        _lib.check(self.lib.crucible_attention_prefill_paged(
            _ptr(q), _dtype(q, "q"), _ptr(k_pool), _ptr(v_pool), _ptr(out), _dtype(out, "out"),
            _ptr(page_table), rows, n_head, n_kv_head, head_dim, n_layer, layer, kv_dim, max_seq,
            _ptr(params), self._stream()))

    def attention_prefill_packed(self, q, k_pool, v_pool, out, tables, owners, positions, rows,
                                 table_stride, n_head, n_kv_head, head_dim, n_layer, layer,
                                 kv_dim, max_seq):
        """gpu.rs:1551-1604: row r of request owners[r] at position positions[r]."""
        _need(q, "q", numel=rows * n_head * head_dim)
        _need(out, "out", numel=rows * n_head * head_dim)
        _need(tables, "tables", dtype=torch.int32)
        _need(owners, "owners", dtype=torch.int32, numel=rows)
        _need(positions, "positions", dtype=torch.int32, numel=rows)
        _lib.check(self.lib.crucible_attention_prefill_packed(
            _ptr(q), _dtype(q, "q"), _ptr(k_pool), _ptr(v_pool), _ptr(out), _dtype(out, "out"),
            _ptr(tables), _ptr(owners), _ptr(positions), rows, table_stride, n_head, n_kv_head,
            head_dim, n_layer, layer, kv_dim, max_seq, self._stream()))

    def attention_prefill_tiled(self, q, k_pool, v_pool, current_k, current_v, out, tables,
                                segments, requests, max_chunk, table_stride, n_head, n_kv_head,
                                head_dim, n_layer, layer, kv_dim, hybrid=False,
                                score_capacity=0):
        """gpu.rs:1606-1751: segments {packed_start, chunk_len, absolute_start, table_index}."""
        _need(segments, "segments", dtype=torch.int32, numel=4 * requests)
        _need(tables, "tables", dtype=torch.int32, numel=requests * table_stride)
        _need(q, "q", numel=max_chunk * n_head * head_dim)
        _need(out, "out", numel=max_chunk * n_head * head_dim)
        _lib.check(self.lib.crucible_attention_prefill_tiled(
            _ptr(q), _dtype(q, "q"), _ptr(k_pool), _ptr(v_pool), _ptr(current_k),
            _ptr(current_v), _ptr(out), _dtype(out, "out"), _ptr(tables), _ptr(segments),
            requests, max_chunk, table_stride, n_head, n_kv_head, head_dim, n_layer, layer,
            kv_dim, int(bool(hybrid)), score_capacity, self._stream()))

    def attention_prefill(self, q, k_cache, v_cache, out, rows, n_head, n_kv_head, head_dim,
                          max_seq, cache_stride, layer_base, pos_offset):
        """gpu.rs:1886-1934: contiguous cache, row r at position pos_offset + r."""
        _need(q, "q", numel=rows * n_head * head_dim)
        _need(out, "out", numel=rows * n_head * head_dim)
        _lib.check(self.lib.crucible_attention_prefill(
            _ptr(q), _dtype(q, "q"), _ptr(k_cache), _ptr(v_cache), _ptr(out), _dtype(out, "out"),
            rows, n_head, n_kv_head, head_dim, max_seq, cache_stride, layer_base, pos_offset,
            self._stream()))

    # ------------------------------------------------------------- decode-step glue
    def linear_f64acc(self, x, w, out, *, norm_w=None, eps=1e-6, resid=None, prefetch=None):
        """out = [resid +] f32(f64-accumulated h . w^T), h = x or rmsnorm(x, norm_w)
        (ops.rs:17-32 matvec, :39-52 rmsnorm). x [rows][k_in] f32, w [n_out][k_in] fp16,
        out (and resid) [rows][n_out] f32; resid may be out itself. prefetch: a contiguous
        device tensor the next kernel reads (its next projection's weights), fetched into
        the last-level cache during this product (crucible_linear_f64acc_prefetch)."""
        rows, k_in = x.shape
        n_out = w.shape[0]
        _need(x, "x", dtype=torch.float32)
        _need(w, "w", dtype=torch.float16, numel=n_out * k_in)
        _need(out, "out", dtype=torch.float32, numel=rows * n_out)
        if norm_w is not None:
            _need(norm_w, "norm_w", dtype=torch.float32, numel=k_in)
        if resid is not None:
            _need(resid, "resid", dtype=torch.float32, numel=rows * n_out)
        args = (_ptr(x), k_in, _ptr(norm_w) if norm_w is not None else None, float(eps),
                _ptr(w), n_out, k_in, _ptr(resid) if resid is not None else None, _ptr(out),
                n_out, rows)
        if prefetch is None:
            _lib.check(self.lib.crucible_linear_f64acc(*args, self._stream()))
        else:
            _lib.check(self.lib.crucible_linear_f64acc_prefetch(
                *args, *_prefetch_region(prefetch), self._stream()))

    def linear_swiglu_f64acc(self, x, w_gate, w_up, out, *, norm_w=None, eps=1e-6,
                             prefetch=None):
        """out = silu(g) * u with g, u the f64-accumulated projections of
        rmsnorm(x, norm_w) (or x) by w_gate and w_up (model.rs:252-262). prefetch: as for
        linear_f64acc."""
        rows, k_in = x.shape
        hidden = w_gate.shape[0]
        _need(x, "x", dtype=torch.float32)
        _need(w_gate, "w_gate", dtype=torch.float16, numel=hidden * k_in)
        _need(w_up, "w_up", dtype=torch.float16, numel=hidden * k_in)
        _need(out, "out", dtype=torch.float32, numel=rows * hidden)
        if norm_w is not None:
            _need(norm_w, "norm_w", dtype=torch.float32, numel=k_in)
        args = (_ptr(x), k_in, _ptr(norm_w) if norm_w is not None else None, float(eps),
                _ptr(w_gate), _ptr(w_up), hidden, k_in, _ptr(out), hidden, rows)
        if prefetch is None:
            _lib.check(self.lib.crucible_linear_swiglu_f64acc(*args, self._stream()))
        else:
            _lib.check(self.lib.crucible_linear_swiglu_f64acc_prefetch(
                *args, *_prefetch_region(prefetch), self._stream()))

    def rmsnorm_rows(self, x, w, out, eps=1e-6):
        """ops.rs:39-52 on every row of x [rows][n]."""
        rows, n = x.shape
        _need(x, "x", dtype=torch.float32)
        _need(w, "w", dtype=torch.float32, numel=n)
        _need(out, "out", dtype=torch.float32, numel=rows * n)
        _lib.check(self.lib.crucible_rmsnorm_rows(_ptr(x), n, _ptr(w), float(eps), _ptr(out), n,
                                                  rows, n, self._stream()))

    def rope_split_qkv(self, qkv, q, k, v, cos, sin, positions, n_head, n_kv_head,
                       head_dim=64):
        """Split [q | k | v] rows and rotate q, k at positions[row] (ops.rs:124-135); cos/sin
        tables [max_pos][head_dim/2]."""
        rows, ld = qkv.shape
        _need(qkv, "qkv", dtype=torch.float32)
        _need(q, "q", dtype=torch.float32, numel=rows * n_head * head_dim)
        _need(k, "k", dtype=torch.float32, numel=rows * n_kv_head * head_dim)
        _need(v, "v", dtype=torch.float32, numel=rows * n_kv_head * head_dim)
        _need(cos, "cos", dtype=torch.float32)
        _need(sin, "sin", dtype=torch.float32, numel=cos.numel())
        _need(positions, "positions", dtype=torch.int32, numel=rows)
        _lib.check(self.lib.crucible_rope_split_qkv(
            _ptr(qkv), ld, _ptr(q), _ptr(k), _ptr(v), _ptr(cos), _ptr(sin), _ptr(positions), rows,
            n_head, n_kv_head, head_dim, cos.shape[0], self._stream()))

    # ------------------------------------------------------------- greedy selection
    def argmax_rows(self, x, out, rows, cols):
        """gpu.rs:562-580 with the host rule of sampling.rs:141-150: ties to the lowest
        index, NaN never wins (a NaN at index 0 yields 0)."""
        _need(x, "x", dtype=torch.float32, numel=rows * cols)
        _need(out, "out", dtype=torch.int32, numel=rows)
        _lib.check(self.lib.crucible_argmax_rows(_ptr(x), _ptr(out), rows, cols, self._stream()))

    def greedy_advance(self, logits, emb, x, tokens, history, step, positions, lens, done):
        """The greedy step's tail on the device (argmax_rows at gpu_model.rs:1586, the
        positions/lengths upload_batch sends, the next step's embed_batch at :1401):
        tokens = argmax(logits) by the argmax_rows rule, history[step] = tokens,
        positions += 1, lens += 1, x = emb[tokens], step += 1. logits [rows][cols] f32,
        emb [cols][n_embd] f32, x [rows][n_embd] f32, history [max_steps][rows] int32,
        step int64 [1], done int32/uint32 [1] (0 between calls)."""
        rows, cols = logits.shape
        n_embd = emb.shape[1]
        _need(logits, "logits", dtype=torch.float32)
        _need(emb, "emb", dtype=torch.float32, numel=cols * n_embd)
        _need(x, "x", dtype=torch.float32, numel=rows * n_embd)
        for t, nm in ((tokens, "tokens"), (positions, "positions"), (lens, "lens")):
            _need(t, nm, dtype=torch.int32, numel=rows)
        _need(history, "history", dtype=torch.int32)
        if history.dim() != 2 or history.shape[1] != rows:
            raise CrucibleError(_lib.ERR_INVALID, "history must be [max_steps][rows]")
        _need(step, "step", dtype=torch.int64, numel=1)
        _need(done, "done", numel=1)
        if done.element_size() != 4:
            raise CrucibleError(_lib.ERR_INVALID, "done must be a 4-byte counter")
        _lib.check(self.lib.crucible_greedy_advance(
            _ptr(logits), rows, cols, _ptr(emb), n_embd, _ptr(x), n_embd, _ptr(tokens),
            _ptr(history), _ptr(step), history.shape[0], _ptr(positions), _ptr(lens), _ptr(done),
            self._stream()))

"""Synthetic inputs for the benchmark configurations.

Metadata (lengths, page tables, segments) is drawn on the host from
``numpy.random.default_rng(seed)``; tensor values are N(0,1) drawn on the device with a
seeded ``torch.Generator`` and rounded to fp16 where the config stores fp16. Seeds are
``20260908 + config_index``. Every config keeps the reference geometry: 16-token pages,
pools of [n_pages][n_layer][16][kv_dim], one table row per sequence.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from .gpu import pool_elems
from ._lib import PAGE_TOKENS

BASE_SEED = 20260908


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)


@dataclass
class DecodeConfig:
    """Paged decode over `batch` sequences (configs 2 and 3)."""
    name: str
    batch: int
    n_head: int
    n_kv_head: int
    n_layer: int
    n_pages: int
    max_seq: int                      # table capacity in tokens
    lens: np.ndarray                  # attention length per sequence (includes the appended token)
    tables: np.ndarray                # [batch, table_stride] int32
    head_dim: int = 64
    seed: int = BASE_SEED
    extra: dict = field(default_factory=dict)

    @property
    def kv_dim(self) -> int:
        return self.n_kv_head * self.head_dim

    @property
    def table_stride(self) -> int:
        return self.tables.shape[1]

    def kv_bytes_per_layer(self) -> int:
        """Algorithmic KV bytes one decode launch reads: sum_b len_b * 2 (K,V) * kv_dim * 2 B."""
        return int(self.lens.astype(np.int64).sum()) * 2 * self.kv_dim * 2

    def io_bytes_per_layer(self) -> int:
        """Query in (fp16), output out (f32), tables and lengths."""
        b = self.batch
        return b * self.n_head * self.head_dim * (2 + 4) + self.tables.nbytes + 4 * b


def _disjoint_tables(rng, n_pages: int, lens, stride: int, offset: int = 0) -> np.ndarray:
    perm = rng.permutation(n_pages).astype(np.int32)
    tables = np.zeros((len(lens), stride), np.int32)
    cur = offset
    for b, length in enumerate(lens):
        need = ceil_div(int(length), PAGE_TOKENS)
        tables[b, :need] = perm[cur:cur + need]
        cur += need
    if cur > n_pages:
        raise ValueError("pool too small for the requested lengths")
    return tables


def config2_decode_b1(n_kv_head: int = 3, seed: int = BASE_SEED + 1) -> DecodeConfig:
    """Batch-1 paged decode: ctx 1024, 4096-page pool, table = 64 pages of a seeded permutation."""
    rng = np.random.default_rng(seed)
    lens = np.array([1024], np.int32)
    tables = _disjoint_tables(rng, 4096, lens, 64)
    return DecodeConfig("decode-b1-ctx1024", 1, 12, n_kv_head, 12, 4096, 1024, lens, tables,
                        seed=seed)


def config3_decode_b16(n_kv_head: int = 3, seed: int = BASE_SEED + 2,
                       rotation: int = 0) -> DecodeConfig:
    """Continuous-batching decode at batch 16, 8192-page pool, context U[64, 2048].

    Existing context lengths are U[64, 2047]; each step appends one token, so the
    attention length is len + 1 in [65, 2048] and the table stride is 128 pages.
    ``rotation`` selects one of several disjoint batches in the same pool (used to
    keep consecutive benchmark steps out of the 256 MB last-level cache).
    """
    rng = np.random.default_rng(seed + 1000 * rotation)
    existing = rng.integers(64, 2048, size=16).astype(np.int32)
    lens = existing + 1
    tables = np.zeros((16, 128), np.int32)
    cfg = DecodeConfig("decode-b16-ctx64-2048-12L", 16, 12, n_kv_head, 12, 8192, 2048, lens,
                       tables, seed=seed)
    cfg.extra["positions"] = existing.copy()   # append position of the new token
    return cfg


def rotation_tables(cfgs: list[DecodeConfig], seed: int) -> None:
    """Give each rotation its own disjoint page set drawn from one pool permutation."""
    rng = np.random.default_rng(seed)
    n_pages = cfgs[0].n_pages
    perm = rng.permutation(n_pages).astype(np.int32)
    cur = 0
    for cfg in cfgs:
        for b, length in enumerate(cfg.lens):
            need = ceil_div(int(length), PAGE_TOKENS)
            if cur + need > n_pages:
                raise ValueError("pool too small for the rotation set")
            cfg.tables[b, :] = 0
            cfg.tables[b, :need] = perm[cur:cur + need]
            cur += need


@dataclass
class PrefillConfig:
    """Causal prefill over packed sequences (configs 1 and 4)."""
    name: str
    n_head: int
    n_kv_head: int
    seq_lens: np.ndarray              # per sequence
    n_layer: int = 1
    head_dim: int = 64
    seed: int = BASE_SEED
    tables: np.ndarray | None = None  # [n_seq, stride]
    n_pages: int = 0

    @property
    def kv_dim(self) -> int:
        return self.n_kv_head * self.head_dim

    @property
    def rows(self) -> int:
        return int(self.seq_lens.sum())

    @property
    def cu_seqlens(self) -> np.ndarray:
        return np.concatenate([[0], np.cumsum(self.seq_lens)]).astype(np.int32)

    def flops(self) -> int:
        """4 * head_dim * n_head * sum_i L_i (L_i + 1) / 2 (visible pairs only)."""
        pairs = sum(int(L) * (int(L) + 1) // 2 for L in self.seq_lens)
        return 4 * self.head_dim * self.n_head * pairs


def _prefill_tables(rng, seq_lens, n_pages=None):
    pages = [ceil_div(int(L), PAGE_TOKENS) for L in seq_lens]
    stride = max(pages)
    n_pages = n_pages or sum(pages) + 8
    perm = rng.permutation(n_pages).astype(np.int32)
    tables = np.zeros((len(seq_lens), stride), np.int32)
    cur = 0
    for i, n in enumerate(pages):
        tables[i, :n] = perm[cur:cur + n]
        cur += n
    return tables, n_pages


def config1_prefill(n_kv_head: int = 12, seed: int = BASE_SEED + 0) -> PrefillConfig:
    """Single-sequence causal prefill, 120m shape: 12 heads, seq 512 (MHA as the SDPA call)."""
    rng = np.random.default_rng(seed)
    cfg = PrefillConfig("prefill-120m-seq512", 12, n_kv_head, np.array([512], np.int32), seed=seed)
    cfg.tables, cfg.n_pages = _prefill_tables(rng, cfg.seq_lens)
    return cfg


def config4_packed(seed: int = BASE_SEED + 3) -> PrefillConfig:
    """Packed varlen prefill, 350m shape: 16/4 heads, 8 sequences of U[32, 512] tokens."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(32, 513, size=8).astype(np.int32)
    cfg = PrefillConfig("packed-350m-8seq", 16, 4, lens, seed=seed)
    cfg.tables, cfg.n_pages = _prefill_tables(rng, lens)
    return cfg


def prefill_sequences(name: str, seq_lens, n_head: int, n_kv_head: int,
                      seed: int = BASE_SEED + 5) -> PrefillConfig:
    """Causal prefill of the given sequences (packed when more than one), for the scaling
    measurements beside configs 1 and 4."""
    rng = np.random.default_rng(seed)
    lens = np.asarray(seq_lens, np.int32)
    cfg = PrefillConfig(name, n_head, n_kv_head, lens, seed=seed)
    cfg.tables, cfg.n_pages = _prefill_tables(rng, lens)
    return cfg


def device_normal(shape, dtype, seed: int, device) -> torch.Tensor:
    """N(0,1) on the device from a seeded generator, cast (RNE) to dtype."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    x = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    return x.to(dtype)


def make_pools(n_pages: int, n_layer: int, kv_dim: int, seed: int, device):
    """K and V pools, fp16 N(0,1) everywhere (the V block order is irrelevant for iid data)."""
    n = pool_elems(n_pages, n_layer, kv_dim)
    k = device_normal((n,), torch.float16, seed, device)
    v = device_normal((n,), torch.float16, seed + 1, device)
    return k, v

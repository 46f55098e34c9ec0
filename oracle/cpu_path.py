"""The reference's CPU attention path, timed as bench.py's cpu_baseline -- TEST INFRASTRUCTURE.

Only ``bench.py``'s cpu_baseline leg (and tests) may import this module; the product never
does. It issues the same PyTorch call the reference's Python model uses for attention,
``torch.nn.functional.scaled_dot_product_attention`` (model.py:205-211 of the reference,
``is_causal`` for prefill, ``enable_gqa`` when n_head > n_kv_head), on fp32 CPU tensors.
Paged decode gathers each sequence's pages by its table first (the gather the paged
engine does implicitly, engine/kernels/kernels.cu:1741-1839 reads ``table[pos >> 4]``),
and the per-step KV append is the row scatter of engine/kernels/kernels.cu:1713-1731.

The pool here is the reference's f32 layout [page][layer][16][kv_dim] holding the
fp16-representable values the GPU pools hold, widened to f32.
"""
from __future__ import annotations

import os
import time

import numpy as np
import torch
import torch.nn.functional as F

PAGE_TOKENS = 16


def threads() -> int:
    """Use every host core this process may run on (set once, reported with the result)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        n = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit():
        n = min(n, int(omp))
    torch.set_num_threads(max(1, n))
    return torch.get_num_threads()


class DecodeBatchCPU:
    """One continuous-batching decode step over all layers, on the CPU.

    ``lens[b]`` includes the token appended this step at position ``lens[b] - 1``.
    """

    def __init__(self, lens, n_layer: int, n_head: int, n_kv_head: int, head_dim: int = 64,
                 seed: int = 0):
        self.lens = np.asarray(lens, np.int64)
        self.n_layer, self.n_head, self.n_kv, self.hd = n_layer, n_head, n_kv_head, head_dim
        self.kv_dim = n_kv_head * head_dim
        g = torch.Generator().manual_seed(seed)
        pages = [-(-int(n) // PAGE_TOKENS) for n in self.lens]
        n_pages = sum(pages)
        perm = torch.randperm(n_pages, generator=g)
        self.tables = []
        cur = 0
        for n in pages:
            self.tables.append(perm[cur:cur + n].clone())
            cur += n
        shape = (n_pages, n_layer, PAGE_TOKENS, self.kv_dim)
        self.k_pool = torch.randn(shape, generator=g).half().float()
        self.v_pool = torch.randn(shape, generator=g).half().float()
        b = len(self.lens)
        self.q = torch.randn((n_layer, b, n_head, 1, head_dim), generator=g).half().float()
        self.src_k = torch.randn((n_layer, b, self.kv_dim), generator=g)
        self.src_v = torch.randn((n_layer, b, self.kv_dim), generator=g)

    def step(self) -> list[torch.Tensor]:
        outs = []
        for layer in range(self.n_layer):
            for b, n in enumerate(self.lens):
                pos = int(n) - 1
                page = self.tables[b][pos // PAGE_TOKENS]
                self.k_pool[page, layer, pos % PAGE_TOKENS] = self.src_k[layer, b].half().float()
                self.v_pool[page, layer, pos % PAGE_TOKENS] = self.src_v[layer, b].half().float()
            for b, n in enumerate(self.lens):
                n = int(n)
                t = self.tables[b]
                k = self.k_pool[t, layer].reshape(-1, self.kv_dim)[:n]
                v = self.v_pool[t, layer].reshape(-1, self.kv_dim)[:n]
                k = k.view(n, self.n_kv, self.hd).transpose(0, 1).unsqueeze(0)
                v = v.view(n, self.n_kv, self.hd).transpose(0, 1).unsqueeze(0)
                q = self.q[layer, b].unsqueeze(0)  # [1, H, 1, hd]
                outs.append(F.scaled_dot_product_attention(
                    q, k, v, enable_gqa=self.n_head != self.n_kv))
        return outs


class PrefillCPU:
    """Causal prefill of packed sequences: one SDPA(is_causal) call per sequence."""

    def __init__(self, seq_lens, n_head: int, n_kv_head: int, head_dim: int = 64, seed: int = 0):
        g = torch.Generator().manual_seed(seed)
        self.n_head, self.n_kv = n_head, n_kv_head
        self.seqs = []
        for n in seq_lens:
            n = int(n)
            q = torch.randn((1, n_head, n, head_dim), generator=g)
            k = torch.randn((1, n_kv_head, n, head_dim), generator=g)
            v = torch.randn((1, n_kv_head, n, head_dim), generator=g)
            self.seqs.append((q, k, v))

    def step(self) -> list[torch.Tensor]:
        return [F.scaled_dot_product_attention(q, k, v, is_causal=True,
                                               enable_gqa=self.n_head != self.n_kv)
                for q, k, v in self.seqs]


def time_bounded(fn, seconds: float, min_reps: int = 3, warmup: int = 1):
    """Run fn at least min_reps times and until `seconds` have passed; return (reps, s/rep)."""
    for _ in range(warmup):
        fn()
    reps = 0
    t0 = time.perf_counter()
    while True:
        fn()
        reps += 1
        dt = time.perf_counter() - t0
        if reps >= min_reps and dt >= seconds:
            return reps, dt / reps

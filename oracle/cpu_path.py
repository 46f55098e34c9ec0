"""The reference's CPU attention path, timed as bench.py's cpu_baseline -- TEST INFRASTRUCTURE.

Only ``bench.py``'s cpu_baseline leg (and tests) may import this module; the product never
does. It issues the same PyTorch call the reference's Python model uses for attention,
``torch.nn.functional.scaled_dot_product_attention`` (model.py:205-211 of the reference,
``is_causal`` for prefill, ``enable_gqa`` when n_head > n_kv_head), on fp32 CPU tensors.
Paged decode gathers each sequence's pages by its table first (the gather the paged
engine does implicitly, engine/kernels/kernels.cu:1741-1839 reads ``table[pos >> 4]``),
and the per-step KV append is the row scatter of engine/kernels/kernels.cu:1713-1731.

The pool here is the reference's f32 layout [page][layer][16][kv_dim] holding the
fp16-representable values the GPU pools hold, widened to f32. bench.py hands in the very
values its GPU run used (host copies of the device pools' pages, queries and appended rows),
so both sides time the same bytes. Timing follows the plan the baseline states: 5 untimed
warmup repetitions, then the median of at least 20 timed repetitions.
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

    ``lens[b]`` includes the token appended this step at position ``lens[b] - 1``. The
    inputs are the GPU run's: ``k_pages``/``v_pages`` [n_pages][n_layer][16][kv_dim] (fp16
    values, reference element order), ``tables`` [batch][>= pages] into them, ``q``
    [n_layer][batch][n_head * head_dim] and the appended rows ``src_k``/``src_v``
    [n_layer][batch][kv_dim] (f32, rounded to fp16 when stored, as the GPU append does).
    """

    def __init__(self, lens, n_layer: int, n_head: int, n_kv_head: int, k_pages, v_pages,
                 tables, q, src_k, src_v, head_dim: int = 64):
        self.lens = np.asarray(lens, np.int64)
        self.n_layer, self.n_head, self.n_kv, self.hd = n_layer, n_head, n_kv_head, head_dim
        self.kv_dim = n_kv_head * head_dim
        pages = [-(-int(n) // PAGE_TOKENS) for n in self.lens]
        self.tables = [torch.from_numpy(np.asarray(tables[b][:n], np.int64))
                       for b, n in enumerate(pages)]
        self.k_pool = torch.from_numpy(np.asarray(k_pages, np.float16)).float()
        self.v_pool = torch.from_numpy(np.asarray(v_pages, np.float16)).float()
        b = len(self.lens)
        self.q = torch.from_numpy(np.asarray(q, np.float16)).float().reshape(
            n_layer, b, n_head, 1, head_dim)
        self.src_k = torch.from_numpy(np.asarray(src_k, np.float32))
        self.src_v = torch.from_numpy(np.asarray(src_v, np.float32))

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
    """Causal prefill of packed sequences: one SDPA(is_causal) call per sequence, on the GPU
    run's packed rows q [rows][n_head * head_dim] and k, v [rows][n_kv_head * head_dim]."""

    def __init__(self, seq_lens, n_head: int, n_kv_head: int, q, k, v, head_dim: int = 64):
        self.n_head, self.n_kv = n_head, n_kv_head
        self.seqs = []
        q = torch.from_numpy(np.asarray(q, np.float32))
        k = torch.from_numpy(np.asarray(k, np.float32))
        v = torch.from_numpy(np.asarray(v, np.float32))
        start = 0
        for n in seq_lens:
            n = int(n)
            sl = slice(start, start + n)
            self.seqs.append((
                q[sl].reshape(n, n_head, head_dim).transpose(0, 1).unsqueeze(0).contiguous(),
                k[sl].reshape(n, n_kv_head, head_dim).transpose(0, 1).unsqueeze(0).contiguous(),
                v[sl].reshape(n, n_kv_head, head_dim).transpose(0, 1).unsqueeze(0).contiguous()))
            start += n

    def step(self) -> list[torch.Tensor]:
        return [F.scaled_dot_product_attention(q, k, v, is_causal=True,
                                               enable_gqa=self.n_head != self.n_kv)
                for q, k, v in self.seqs]


def time_median(fn, seconds: float, min_reps: int = 20, warmup: int = 5):
    """5 untimed warmup calls, then timed calls until at least min_reps have run and
    `seconds` have passed; returns (reps, median seconds per call)."""
    for _ in range(warmup):
        fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < min_reps or time.perf_counter() - t_start < seconds:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return len(times), float(np.median(times))


def cpu_model() -> str:
    """The host CPU's model name (lscpu's "Model name", read from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:  # pragma: no cover
        pass
    return "unknown"

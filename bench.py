#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path (one JSON line on stdout).

Headline workload: continuous-batching paged decode at batch 16,
120m preset geometry (12 query heads, 3 KV heads of head_dim 64, 12 layers), fp16 KV in
16-token pages from an 8192-page pool, context lengths seeded U[64, 2048]. One step is,
for every layer, the KV append of one new token per sequence (K and V, f32 -> fp16) and
paged decode attention over len + 1 keys, done by one fused launch per layer. The
12-layer step is captured once per batch in a HIP graph and replayed, so the timed
region measures the device work, not Python.

Consecutive steps rotate over several disjoint batches drawn from the same pool, so a
step never finds its KV pages in the 256 MB last-level cache from the previous step.

value  = algorithmic bytes of the whole step (KV pages read, appended rows, queries,
         outputs, tables) / wall time of the timed steps, in GB/s.
roofline = the one kernel of the step (fused append + paged decode attention): algorithmic
         bytes per launch over its average launch duration, HIP events on the replay stream.
cpu_baseline = the reference's CPU attention path (gather + torch SDPA, fp32) on the host
         cores, on a bounded sample of the same workload.
extras = the same step as the reference's three launches per layer and as attention
         alone, batch-1 decode (config 2), the MHA stress variant of config 3, the causal
         (config 1) and packed (config 4) prefill kernels, prefill of 2k..8k-token
         sequences (the MFMA rate once a launch is compute-heavy), and end-to-end greedy
         decoding of the random-init 120m model at batch 16 (config 5, tok/s).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, TFLOP/s
METRIC = "paged-attn decode HBM GB/s (% peak); prefill attn TFLOP/s; 120M tok/s at b16"


MFMA_PEAK_CLOCK_MHZ = 2400.0  # the clock the published dense MFMA peak assumes

_SMI = {}


def power_envelope() -> dict:
    """The power and clock envelope of GPU 0 at this moment, from amdsmi: enforced power cap
    and maximum gfx clock (what the reference records with every benchmark, nvidia-smi's
    enforced.power.limit and clocks.max.sm; engine/src/gpu.rs:2159-2186, main.rs:1285-1305),
    plus the current and recently averaged gfx clock, socket power and hotspot temperature.
    Fields that the driver does not report are left out; an unavailable amdsmi gives
    {"error": ...}. Powers in W, clocks in MHz, temperatures in C."""
    try:
        import amdsmi
        if "h" not in _SMI:
            amdsmi.amdsmi_init()
            _SMI["h"] = amdsmi.amdsmi_get_processor_handles()[0]
        h = _SMI["h"]
    except Exception as e:  # noqa: BLE001 - the envelope is a report, never a failure
        return {"error": f"amdsmi unavailable: {e}"[:200]}
    out = {}

    def num(v):
        return v if isinstance(v, (int, float)) and v not in (0xFFFF, 0xFFFFFFFF) else None

    try:
        clk = amdsmi.amdsmi_get_clock_info(h, amdsmi.AmdSmiClkType.GFX)
        out["gfx_clk_mhz"] = num(clk.get("clk"))
        out["gfx_clk_max_mhz"] = num(clk.get("max_clk"))
    except Exception as e:  # noqa: BLE001
        out["clock_error"] = str(e)[:120]
    try:
        m = amdsmi.amdsmi_get_gpu_metrics_info(h)
        out["gfx_clk_avg_mhz"] = num(m.get("average_gfxclk_frequency"))
        out["socket_power_w"] = num(m.get("current_socket_power")) or num(
            m.get("average_socket_power"))
        out["hotspot_c"] = num(m.get("temperature_hotspot"))
    except Exception as e:  # noqa: BLE001
        out["metrics_error"] = str(e)[:120]
    try:
        cap = amdsmi.amdsmi_get_power_cap_info(h)
        pc = num(cap.get("power_cap"))
        out["power_cap_w"] = round(pc / 1e6, 1) if pc and pc > 1e5 else pc  # reported in uW
    except Exception as e:  # noqa: BLE001
        out["power_cap_error"] = str(e)[:120]
    return {k: v for k, v in out.items() if v is not None}


def clock_scaled_fraction(tflops: float, env: dict):
    """The MFMA fraction against the peak at the clock the envelope read (the published
    2.5 PFLOP/s assumes 2.4 GHz), or None without a clock reading."""
    mhz = env.get("gfx_clk_avg_mhz") or env.get("gfx_clk_mhz")
    if not mhz:
        return None
    return round(tflops / (MFMA_F16_PEAK_TFLOPS * mhz / MFMA_PEAK_CLOCK_MHZ), 5)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=300)
    p.add_argument("--warmup", type=int, default=30)
    p.add_argument("--kv-heads", type=int, default=3, help="3 = 120m preset (GQA), 12 = MHA")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extras", action="store_true")
    p.add_argument("--extras", default="decode,prefill,pscale,e2e",
                   help="comma list of extra groups to run: decode (the other decode "
                        "shapes), prefill (configs 1 and 4), pscale (prefill of 2k..8k-token "
                        "sequences), e2e (config 5), scale (pscale plus the fused decode at "
                        "batch 32..256 with config 3's length distribution; not in the "
                        "default set)")
    p.add_argument("--copy-probe", action="store_true",
                   help="also run 5 more plain 256 MiB device copies (PMC traffic calibration)")
    p.add_argument("--phases", nargs="?", const="decode", choices=("decode", "config4", "config1"),
                   help="diagnostic: run config 3 (decode, the default), config 4 (the "
                        "16-row LDS prefill) or config 1 (the register-direct prefill) on the "
                        "stamped twin of the library "
                        "(libcrucible_attn_stamps.so) and print where a launch's time goes, "
                        "per phase, instead of the bench line")
    p.add_argument("--phase-reps", type=int, default=28,
                   help="--phases: replayed steps whose last launch is read")

    return p.parse_args()


# ---------------------------------------------------------------- decode workload

class DecodeBench:
    """Config 3 (or 2) on the device: pools, per-layer inputs, one graph per rotation."""

    def __init__(self, gpu, dev, *, batch, n_head, n_kv_head, n_layer, n_pages, max_seq,
                 rotations, seed, fixed_lens=None):
        import numpy as np
        import torch

        from crucible_amd import workloads as W
        from crucible_amd.gpu import pool_elems

        self.gpu, self.dev = gpu, dev
        self.batch, self.n_head, self.n_kv, self.n_layer = batch, n_head, n_kv_head, n_layer
        self.kv_dim = n_kv_head * 64
        self.max_seq = max_seq
        self.stride = max_seq // 16
        rng = np.random.default_rng(seed)
        # draw batches until the pool is used up (at most `rotations`)
        self.lens, self.tables = [], []
        perm = rng.permutation(n_pages).astype(np.int32)
        cur = 0
        for _ in range(rotations):
            if fixed_lens is not None:
                existing = np.asarray(fixed_lens, np.int32) - 1
            else:
                existing = rng.integers(64, max_seq, size=batch).astype(np.int32)
            lens = existing + 1
            need = [W.ceil_div(int(n), 16) for n in lens]
            if cur + sum(need) > n_pages:
                break
            tab = np.zeros((batch, self.stride), np.int32)
            for b, k in enumerate(need):
                tab[b, :k] = perm[cur:cur + k]
                cur += k
            self.lens.append(lens)
            self.tables.append(tab)
        self.rotations = len(self.lens)
        n = pool_elems(n_pages, n_layer, self.kv_dim)
        self.k_pool = W.device_normal((n,), torch.float16, seed + 11, dev)
        self.v_pool = W.device_normal((n,), torch.float16, seed + 12, dev)
        self.q = W.device_normal((n_layer, batch, n_head * 64), torch.float16, seed + 13, dev)
        self.src_k = W.device_normal((n_layer, batch, self.kv_dim), torch.float32, seed + 14, dev)
        self.src_v = W.device_normal((n_layer, batch, self.kv_dim), torch.float32, seed + 15, dev)
        self.out = torch.zeros((n_layer, batch, n_head * 64), dtype=torch.float32, device=dev)
        self.d_tables = [torch.from_numpy(t).to(dev) for t in self.tables]
        self.d_lens = [torch.from_numpy(x).to(dev) for x in self.lens]
        self.d_pos = [torch.from_numpy(x - 1).to(dev) for x in self.lens]
        self.ws = gpu.workspace(batch, n_head, max_seq)

    # algorithmic bytes ----------------------------------------------------------
    def decode_bytes(self, r: int) -> int:
        """One decode launch: K and V of every visible key (fp16), fp16 q, f32 out,
        the used table entries and the lengths."""
        lens = self.lens[r].astype("int64")
        kv = int(lens.sum()) * 2 * self.kv_dim * 2
        pages = int(sum((int(n) + 15) // 16 for n in lens))
        return kv + self.batch * self.n_head * 64 * (2 + 4) + 4 * pages + 4 * self.batch

    def append_bytes(self) -> int:
        """K and V appends of one layer: f32 rows in, fp16 rows out, positions, table reads."""
        return 2 * (self.batch * self.kv_dim * (4 + 2) + 8 * self.batch)

    def step_bytes(self, r: int) -> int:
        return self.n_layer * (self.decode_bytes(r) + self.append_bytes())

    # launches ---------------------------------------------------------------------
    def append(self, r: int, layer: int):
        g = self.gpu
        for src, pool, kind in ((self.src_k, self.k_pool, "k"), (self.src_v, self.v_pool, "v")):
            g.cache_store_rows_paged(src[layer], pool, self.d_tables[r], self.d_pos[r],
                                     self.batch, self.kv_dim, self.stride, self.n_layer, layer,
                                     kind=kind)

    def decode(self, r: int, layer: int):
        self.gpu.attention_decode_paged(
            self.q[layer], self.k_pool, self.v_pool, self.out[layer], self.d_tables[r],
            self.d_lens[r], self.batch, self.n_head, self.n_kv, 64, self.stride, self.n_layer,
            layer, self.kv_dim, self.max_seq, workspace=self.ws)

    def fused(self, r: int, layer: int):
        self.gpu.attention_decode_paged_append(
            self.q[layer], self.src_k[layer], self.src_v[layer], self.k_pool, self.v_pool,
            self.out[layer], self.d_tables[r], self.d_pos[r], self.d_lens[r], self.batch,
            self.n_head, self.n_kv, 64, self.stride, self.n_layer, layer, self.kv_dim,
            self.max_seq, workspace=self.ws)

    def step(self, r: int, mode: str):
        """One 12-layer step: 'fused' (one launch per layer), 'separate' (the reference's
        append K, append V, decode), or 'decode' (attention only)."""
        for layer in range(self.n_layer):
            if mode == "fused":
                self.fused(r, layer)
            elif mode == "separate":
                self.append(r, layer)
                self.decode(r, layer)
            else:
                self.decode(r, layer)

    def capture(self, mode: str):
        """One graph per rotation holding a full step."""
        import torch

        s = torch.cuda.Stream(self.dev)
        s.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(s):
            for r in range(self.rotations):
                self.step(r, mode)
        torch.cuda.current_stream(self.dev).wait_stream(s)
        torch.cuda.synchronize(self.dev)
        graphs = []
        for r in range(self.rotations):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.step(r, mode)
            graphs.append(g)
        torch.cuda.synchronize(self.dev)
        return graphs

    def time_steps(self, graphs, steps: int, warmup: int, bytes_fn=None):
        """Wall time of `steps` graph replays (rotating batches), HIP events on the replay
        stream alongside; returns (ms per step by wall clock, ms per step by events, bytes)."""
        import torch

        for i in range(warmup):
            graphs[i % len(graphs)].replay()
        flush_llc(self.dev)
        torch.cuda.synchronize(self.dev)
        stream = torch.cuda.current_stream(self.dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        bytes_fn = bytes_fn or self.step_bytes
        nbytes = sum(bytes_fn(i % len(graphs)) for i in range(steps))
        t0 = time.perf_counter()
        e0.record(stream)
        for i in range(steps):
            graphs[i % len(graphs)].replay()
        e1.record(stream)
        torch.cuda.synchronize(self.dev)
        wall = time.perf_counter() - t0
        return wall * 1e3 / steps, e0.elapsed_time(e1) / steps, nbytes / steps


def pmc_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary
    (profiles/decode_b16_gqa3_pmc_traffic.txt: FETCH_SIZE and WRITE_SIZE runs scaled by a
    copy kernel of known size), or None unless the summary is for this very kernel built
    from these very sources (its kernel and source_sha lines)."""
    path = os.path.join(ROOT, "profiles", "decode_b16_gqa3_pmc_traffic.txt")
    try:
        fields = dict(line.split(": ", 1) for line in open(path).read().splitlines()
                      if ": " in line and not line.startswith(" "))
    except OSError:
        return None
    if fields.get("kernel", "").strip() != kernel:
        return None
    if fields.get("source_sha", "").strip() != source_sha():
        return None
    return int(fields["traffic_bytes_per_launch"])


def flush_llc(dev):
    """Touch 512 MiB so the 256 MB last-level cache holds nothing of the workload."""
    import torch

    buf = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    buf.fill_(1)
    del buf


# ---------------------------------------------------------------- prefill workloads

def gather_rows(pool, table_row, n, n_layer, layer, kv_dim, v_kind):
    """Rows [0, n) of one sequence from a device pool, reference element order [n][kv_dim]
    (V blocks are stored transposed)."""
    n_pages = -(-n // 16)
    blocks = pool.view(-1, n_layer, 16 * kv_dim)[table_row[:n_pages].long(), layer]
    if v_kind:
        blocks = blocks.view(n_pages, kv_dim, 16).transpose(1, 2)
    return blocks.reshape(n_pages * 16, kv_dim)[:n]


def prefill_runner(gpu, dev, cfg, q_dtype=None):
    """Device inputs of a prefill config and a closure that launches its segment-form
    prefill once (its output tensor is run.out); returns (run, q, k_pool, v_pool, tables)."""
    import numpy as np
    import torch

    from crucible_amd import workloads as W
    from crucible_amd.gpu import pool_elems
    from crucible_amd.paged import segments_from_cu_seqlens

    kv_dim = cfg.kv_dim
    rows = cfg.rows
    stride = cfg.tables.shape[1]
    k_pool = W.device_normal((pool_elems(cfg.n_pages, 1, kv_dim),), torch.float16, cfg.seed + 1, dev)
    v_pool = W.device_normal((pool_elems(cfg.n_pages, 1, kv_dim),), torch.float16, cfg.seed + 2, dev)
    q = W.device_normal((rows, cfg.n_head * 64), q_dtype or torch.float16, cfg.seed + 3, dev)
    out = torch.empty((rows, cfg.n_head * 64), dtype=torch.float32, device=dev)
    seg, max_chunk = segments_from_cu_seqlens(cfg.cu_seqlens)
    d_seg = torch.from_numpy(np.ascontiguousarray(seg)).to(dev)
    d_tab = torch.from_numpy(cfg.tables).to(dev)

    def run():
        gpu.attention_prefill_tiled(q, k_pool, v_pool, None, None, out, d_tab, d_seg,
                                    len(cfg.seq_lens), max_chunk, stride, cfg.n_head,
                                    cfg.n_kv_head, 64, 1, 0, kv_dim)

    run.out = out  # the output rows the launch writes
    return run, q, k_pool, v_pool, d_tab


def bench_prefill(gpu, dev, cfg, launches: int = 50, q_dtype=None, cpu_inputs=None):
    """Time the segment-form prefill kernel (gpu.rs:1606-1751 path) on config 1 or 4:
    `launches` back-to-back launches replayed from one HIP graph (us_per_launch, the
    figure TFLOP/s uses, timed like the decode step), and eager launches each bracketed by
    events (us_per_launch_eager). The query is fp16 (the kernel's MFMA input type) unless
    q_dtype says otherwise."""
    import torch

    run, q, k_pool, v_pool, d_tab = prefill_runner(gpu, dev, cfg, q_dtype)
    kv_dim = cfg.kv_dim
    for _ in range(5):
        run()
    torch.cuda.synchronize(dev)
    stream = torch.cuda.current_stream(dev)
    # eager: every launch bracketed by its own events (includes the launch path)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(launches)]
    for a, b in ev:
        a.record(stream)
        run()
        b.record(stream)
    torch.cuda.synchronize(dev)
    ms = sorted(a.elapsed_time(b) for a, b in ev)
    eager = sum(ms) / len(ms)
    # graph replay of `launches` back-to-back launches, as the decode step is timed
    side = torch.cuda.Stream(dev)
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        run()
    stream.wait_stream(side)
    torch.cuda.synchronize(dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(launches):
            run()
    g.replay()
    torch.cuda.synchronize(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(4):
        g.replay()
    e1.record(stream)
    torch.cuda.synchronize(dev)
    avg = e0.elapsed_time(e1) / (4 * launches)
    del g
    tflops = cfg.flops() / (avg * 1e-3) / 1e12
    env = power_envelope()  # right after the timed replays
    if cpu_inputs is not None:  # the rows this run used, for the CPU baseline beside it
        ks, vs = [], []
        for i, n in enumerate(cfg.seq_lens):
            ks.append(gather_rows(k_pool, d_tab[i], int(n), 1, 0, kv_dim, False))
            vs.append(gather_rows(v_pool, d_tab[i], int(n), 1, 0, kv_dim, True))
        cpu_inputs.update(q=q.float().cpu().numpy(), k=torch.cat(ks).float().cpu().numpy(),
                          v=torch.cat(vs).float().cpu().numpy())
    from crucible_amd import _lib
    p16 = _lib.load().crucible_attn_get_tuning(_lib.TUNE_KEYS["prefill_p16"]) == 1
    return {"workload": cfg.name, "n_head": cfg.n_head, "n_kv_head": cfg.n_kv_head,
            "q_dtype": str(q.dtype).replace("torch.", ""),
            "p_operand": "one fp16 (RNE)" if p16 else "fp16 hi + lo",
            "seq_lens": [int(x) for x in cfg.seq_lens], "flops": cfg.flops(),
            "us_per_launch": round(avg * 1e3, 3),
            "us_per_launch_eager": round(eager * 1e3, 3), "us_median_eager": round(ms[len(ms) // 2] * 1e3, 3),
            "tflops": round(tflops, 3), "frac_of_mfma_f16_peak": round(tflops / MFMA_F16_PEAK_TFLOPS, 5),
            "gfx_clk_mhz": env.get("gfx_clk_avg_mhz") or env.get("gfx_clk_mhz"),
            "frac_of_mfma_f16_peak_at_clock": clock_scaled_fraction(tflops, env)}


# ---------------------------------------------------------------- end to end (config 5)

def bench_e2e(gpu, reps: int = 3):
    """random-init 120m preset, 16 prompts of U[64, 512] seeded token
    ids, 256 greedy tokens each, decode steps replayed from one HIP graph. tok/s counts the
    decode loop only (16 x 255 steps after the prefill's first token). The greedy tokens
    equal the CPU oracle's (tests/test_gpu_e2e.py)."""
    from crucible_amd.gpu_model import PRESET_120M, GpuModel, random_weights, seeded_prompts

    cfg = PRESET_120M
    seed = 20260908 + 4
    model = GpuModel(cfg, random_weights(cfg, seed=seed), max_batch=16, capacity=1024, gpu=gpu)
    prompts = seeded_prompts(seed, 16, 64, 512, cfg.vocab_size)
    runs = []
    for _ in range(reps):
        timing = {}
        model.generate(prompts, 256, timing=timing)
        runs.append(timing)
    # decode_ms times the graph replays of the decode loop (captured once per generate call;
    # a server captures once per process), events on the replay stream; the median run
    t = sorted(runs, key=lambda r: r["decode_ms"])[len(runs) // 2]
    tok_s = 16 * t["decode_steps"] / (t["decode_ms"] * 1e-3)
    # the prefill's median too (the first run also allocates the prompt-sized buffers)
    prefill_ms = sorted(r["prefill_ms"] for r in runs)[len(runs) // 2]
    return {"workload": "config5 greedy decode, random-init 120m (12 layers, 12/3 heads, "
                        "vocab 50257), b16, prompts U[64,512], 256 tokens",
            "tok_per_s": round(tok_s, 1), "ms_per_step": round(t["decode_ms"] / t["decode_steps"], 4),
            "prefill_ms": round(prefill_ms, 3), "decode_steps": t["decode_steps"],
            "runs": len(runs), "ms_per_step_runs": [round(r["decode_ms"] / r["decode_steps"], 4)
                                                    for r in runs],
            "capture_ms": round(t["capture_ms"], 2),
            "precision": "reference (f64-accumulated projections)",
            "reference_published_tok_per_s": 8366}


# ---------------------------------------------------------------- CPU baseline

def cpu_prefill(cfg, inputs, seconds: float):
    """The reference CPU attention for a prefill config (one SDPA(is_causal) per sequence,
    fp32) on the same rows the GPU run used: GFLOP/s on the config's visible-pair FLOPs."""
    from oracle import cpu_path

    cores = cpu_path.threads()
    cpu = cpu_path.PrefillCPU(cfg.seq_lens, cfg.n_head, cfg.n_kv_head, inputs["q"],
                              inputs["k"], inputs["v"])
    reps, s_per = cpu_path.time_median(cpu.step, seconds)
    return {"ms": round(s_per * 1e3, 3), "gflops": round(cfg.flops() / s_per / 1e9, 2),
            "cores": cores, "kind": "port", "cpu_model": cpu_path.cpu_model(),
            "sample": f"median of {reps} full launches after 5 warmups, torch SDPA fp32 per "
                      "sequence on the GPU run's rows"}


def decode_cpu_inputs(bench, r: int = 0):
    """Host copies of what rotation r of a decode bench reads: its pages (compacted, K and V
    in reference element order), remapped tables, queries and appended rows."""
    import numpy as np
    import torch

    lens = bench.lens[r]
    tab = bench.tables[r]
    pages = [-(-int(n) // 16) for n in lens]
    used = np.concatenate([tab[b, :n] for b, n in enumerate(pages)])
    blk = bench.n_layer * 16 * bench.kv_dim
    idx = torch.from_numpy(used.astype(np.int64)).to(bench.dev)
    k = bench.k_pool.view(-1, blk)[idx].view(-1, bench.n_layer, 16, bench.kv_dim)
    v = bench.v_pool.view(-1, blk)[idx].view(-1, bench.n_layer, bench.kv_dim, 16).transpose(2, 3)
    compact = []
    cur = 0
    for n in pages:
        compact.append(np.arange(cur, cur + n))
        cur += n
    return dict(k_pages=k.contiguous().cpu().numpy(), v_pages=v.contiguous().cpu().numpy(),
                tables=compact, q=bench.q.cpu().numpy(), src_k=bench.src_k.cpu().numpy(),
                src_v=bench.src_v.cpu().numpy())


def cpu_decode(bench, seconds: float, r: int = 0):
    """A decode bench's step on the CPU (per layer and sequence: the row append, the page
    gather and torch SDPA, fp32), on the same bytes as the GPU run's rotation r."""
    from oracle import cpu_path

    cores = cpu_path.threads()
    lens = bench.lens[r]
    cpu = cpu_path.DecodeBatchCPU(lens, bench.n_layer, bench.n_head, bench.n_kv,
                                  **decode_cpu_inputs(bench, r))
    reps, s_per_step = cpu_path.time_median(cpu.step, seconds)
    return reps, s_per_step, cores, cpu_path.cpu_model()


def cpu_baseline(bench, seconds: float):
    import torch

    reps, s_per_step, cores, model = cpu_decode(bench, seconds)
    lens = bench.lens[0]
    gbs = bench.step_bytes(0) / s_per_step / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "cpu_model": model, "ms_per_step": round(s_per_step * 1e3, 3),
            "sample": (f"median of {reps} full {bench.n_layer}-layer decode steps of batch 0 "
                       f"after 5 warmups (16 sequences, lens {int(lens.min())}..{int(lens.max())}, "
                       f"the GPU run's own pages, queries and rows): per layer and sequence a row "
                       f"append, a page gather and torch SDPA, fp32, torch {torch.__version__}")}


def copy_bandwidth(dev, mib: int = 256, reps: int = 10):
    """Device-to-device copy of `mib` MiB (HIP's copy kernel), GB/s counting the bytes read
    and written: the measured ceiling beside the 8 TB/s spec."""
    import torch

    src = torch.ones(mib << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    stream = torch.cuda.current_stream(dev)
    e0.record(stream)
    for _ in range(reps):
        dst.copy_(src)
    e1.record(stream)
    torch.cuda.synchronize(dev)
    ms = e0.elapsed_time(e1) / reps
    del src, dst
    return 2 * (mib << 20) / (ms * 1e-3) / 1e9


PHASES = ("unit", "issue", "loads", "compute", "merge", "publish", "counter", "combine")


def decode_phases(gpu, dev, args, log):
    """Per-workgroup phase stamps of the fused config-3 decode launch (the stamped library).

    Each replay of a step graph runs the 12 layer launches back to back; the stamps left
    afterwards are those of the last one. Per workgroup, from its slots (StampSlot in
    attn_decode.hip): start skew (entry against the launch's first entry), unit (entry to
    the workgroup's unit known: the plan entry and the lengths in, or the search done),
    issue (to the page ids in and the K/V loads issued), loads (to wave 0's pages
    resident), compute (wave 0's products issued), merge (to every wave past the LDS
    merge), publish (partial acknowledged, or the output stored for a one-split unit),
    counter (split counter returned) and, for the combining workgroup, combine (output
    stored). `chain` is the launch's first entry to its last stamp.
    """
    import ctypes

    import numpy as np
    import torch

    from crucible_amd import _lib
    from crucible_amd import workloads as W

    fn = gpu.lib.crucible_debug_decode_stamps
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                   ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
    fn.restype = ctypes.c_int
    khz, slots = ctypes.c_int(0), ctypes.c_int(0)
    _lib.check(fn(None, 0, 1, ctypes.byref(khz), ctypes.byref(slots)))
    rows = 8192
    buf = np.zeros((rows, slots.value), np.uint64)

    b16 = DecodeBench(gpu, dev, batch=16, n_head=12, n_kv_head=args.kv_heads, n_layer=12,
                      n_pages=8192, max_seq=2048, rotations=7, seed=W.BASE_SEED + 2)
    graphs = b16.capture("fused")
    ms, ev, _ = b16.time_steps(graphs, 60, 10)
    kernel = decode_kernel_name(gpu, 16, 12, args.kv_heads, 2048, 1)
    log(f"stamped build: {ev * 1e3 / 12:.2f} us per launch (events), kernel {kernel}")
    us_per_tick = 1e3 / khz.value
    launches = []
    for rep in range(args.phase_reps):
        _lib.check(fn(None, 0, 1, ctypes.byref(khz), ctypes.byref(slots)))
        graphs[rep % len(graphs)].replay()
        torch.cuda.synchronize(dev)
        _lib.check(fn(buf.ctypes.data, rows, 0, ctypes.byref(khz), ctypes.byref(slots)))
        launches.append(buf.copy())
    out = summarize_stamps(launches, us_per_tick)
    return {"kernel": kernel, "clock_khz": khz.value, "stamped_us_per_launch": round(ev * 1e3 / 12, 3),
            **out}


def summarize_stamps(launches, us_per_tick: float) -> dict:
    """Phase durations (median, p90, max over workgroups and launches) from stamp rows of
    one launch each (uint64 [rows][10]: StampSlot order, slot 9 the meta word), and the
    phases of each launch's last-finishing workgroup."""
    import numpy as np

    per = {k: [] for k in ("skew",) + PHASES + ("chain",)}
    crit = []
    n_wg = 0
    n_all = len(PHASES)  # 8 phases between 9 time slots
    for buf in launches:
        meta = buf[:, n_all + 1]
        kind = (meta >> np.uint64(52)) & np.uint64(0xF)
        n_active = ((meta >> np.uint64(32)) & np.uint64(0xFFFF)).astype(np.int64)
        last = ((meta >> np.uint64(48)) & np.uint64(1)).astype(bool)
        att = (buf[:, 0] != 0) & (kind == 0) & (buf[:, n_all - 2] != 0)
        n_wg = int(att.sum())
        t = buf[att, :n_all + 1].astype(np.int64)
        multi = n_active[att] > 1
        comb = multi & last[att]
        t0 = t[:, 0].min()
        # a one-split unit stops at the publish slot, a non-combining split at the counter
        # slot (later slots may hold an earlier launch's values)
        end = np.where(comb, t[:, n_all], np.where(multi, t[:, n_all - 1], t[:, n_all - 2]))
        d = np.diff(t, axis=1) * us_per_tick  # slots 0..8 -> the 8 phases
        per["skew"] += list((t[:, 0] - t0) * us_per_tick)
        for i, name in enumerate(PHASES[:n_all - 2]):
            per[name] += list(d[:, i])
        per["counter"] += list(d[multi, n_all - 2])
        per["combine"] += list(d[comb, n_all - 1])
        per["chain"].append(float((end.max() - t0) * us_per_tick))
        w = int(np.argmax(end))
        n_ph = n_all if comb[w] else n_all - 1 if multi[w] else n_all - 2
        crit.append({"skew": round(float((t[w, 0] - t0) * us_per_tick), 2),
                     **{PHASES[i]: round(float(d[w, i]), 2) for i in range(n_ph)}})
    summary = {}
    for k, v in per.items():
        a = np.asarray(v, np.float64)
        summary[k] = {"median_us": round(float(np.median(a)), 3),
                      "p90_us": round(float(np.percentile(a, 90)), 3),
                      "max_us": round(float(a.max()), 3), "n": int(a.size)}
    return {"launches_read": len(launches), "workgroups_per_launch": n_wg,
            "phases": summary, "critical_workgroup": crit[:8]}


PREFILL_PHASES = ("rows", "first_pair", "loop", "merge", "write")


def prefill_phases(gpu, dev, args, log):
    """Per-workgroup phase stamps of a prefill launch on the stamped library: config 4 (the
    16-row LDS kernel) or config 1 (the register-direct kernel). A graph of 12 back-to-back
    launches is replayed; the stamps left are the last launch's. Per workgroup with rows
    (slots of PStampSlot in attn_prefill.hip): start skew, rows (entry to the tile's rows
    resolved; direct form: and the query loads issued), first_pair (LDS form: to the first
    pair of key tiles in LDS, page ids, tile loads and query loads; direct form: to wave 0's
    first key tile in registers), loop (the rest of the tile loop), merge (the states
    merged), write (output stored), and `wait`, the part of first_pair + loop the LDS form's
    wave spent waiting for key tiles (0 in the direct form). Reported over all workgroups
    and over the heaviest (most tile pairs, resp. key tiles), whose chain bounds the launch."""
    import ctypes

    import numpy as np
    import torch

    from crucible_amd import _lib
    from crucible_amd import workloads as W

    fn = gpu.lib.crucible_debug_prefill_stamps
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                   ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
    fn.restype = ctypes.c_int
    khz, slots = ctypes.c_int(0), ctypes.c_int(0)
    _lib.check(fn(None, 0, 1, ctypes.byref(khz), ctypes.byref(slots)))
    rows = 8192
    buf = np.zeros((rows, slots.value), np.uint64)
    direct = args.phases == "config1"
    cfg = W.config1_prefill(n_kv_head=12) if direct else W.config4_packed()
    timing = bench_prefill(gpu, dev, cfg, launches=12)
    log(f"stamped build: {timing['us_per_launch']} us per launch (graph replay)")
    run = prefill_runner(gpu, dev, cfg)[0]
    stream = torch.cuda.current_stream(dev)
    side = torch.cuda.Stream(dev)
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        run()
    stream.wait_stream(side)
    torch.cuda.synchronize(dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(12):
            run()
    us = 1e3 / khz.value
    per = {k: [] for k in ("skew",) + PREFILL_PHASES + ("wait", "chain")}
    heavy = {k: [] for k in ("skew",) + PREFILL_PHASES + ("wait",)}
    n_wg = 0
    for _ in range(args.phase_reps):
        _lib.check(fn(None, 0, 1, ctypes.byref(khz), ctypes.byref(slots)))
        g.replay()
        torch.cuda.synchronize(dev)
        _lib.check(fn(buf.ctypes.data, rows, 0, ctypes.byref(khz), ctypes.byref(slots)))
        live = (buf[:, 0] != 0) & (buf[:, 5] != 0)
        t = buf[live, :6].astype(np.int64)
        wait = buf[live, 6].astype(np.int64)
        pairs = (buf[live, 7] >> np.uint64(48)).astype(np.int64)
        n_wg = int(live.sum())
        t0 = t[:, 0].min()
        d = np.diff(t, axis=1) * us
        hv = pairs == pairs.max()
        for sel, dst in ((np.ones_like(hv), per), (hv, heavy)):
            dst["skew"] += list((t[sel, 0] - t0) * us)
            for i, name in enumerate(PREFILL_PHASES):
                dst[name] += list(d[sel, i])
            dst["wait"] += list(wait[sel] * us)
        per["chain"].append(float((t[:, 5].max() - t0) * us))
    del g

    def stats(dct):
        out = {}
        for k, v in dct.items():
            a = np.asarray(v, np.float64)
            out[k] = {"median_us": round(float(np.median(a)), 3),
                      "p90_us": round(float(np.percentile(a, 90)), 3),
                      "max_us": round(float(a.max()), 3), "n": int(a.size)}
        return out

    p16 = "true" if timing["p_operand"].startswith("one") else "false"
    kernel = (f"prefill_direct_kernel<false, false, {p16}>" if direct
              else f"prefill_kernel<4, 1, false, 4, {p16}>")
    return {"kernel": kernel, "workload": cfg.name,
            "clock_khz": khz.value, "stamped_us_per_launch": timing["us_per_launch"],
            "launches_read": args.phase_reps, "workgroups_per_launch": n_wg,
            "max_pairs": int(pairs.max()), "phases": stats(per), "heaviest": stats(heavy)}


def launch_floor_us(dev, launches: int = 12, reps: int = 50):
    """Time per launch of a one-element fill kernel, `launches` back to back in one HIP
    graph and replayed as the decode step is: what any kernel of a captured step costs
    before it does any work (dispatch, wave launch, end-of-kernel release)."""
    import torch

    x = torch.zeros(1, device=dev)
    stream = torch.cuda.current_stream(dev)
    side = torch.cuda.Stream(dev)
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        x.fill_(1.0)
    stream.wait_stream(side)
    torch.cuda.synchronize(dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(launches):
            x.fill_(1.0)
    for _ in range(5):
        g.replay()
    torch.cuda.synchronize(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        g.replay()
    e1.record(stream)
    torch.cuda.synchronize(dev)
    us = e0.elapsed_time(e1) * 1e3 / (reps * launches)
    del g
    return us


# What the decode kernel is built from: its translation unit and the headers it includes,
# plus the compiler flags the build gives that unit (not the rest of the build script).
DECODE_SOURCES = ("crucible_amd/csrc/attn_decode.hip", "crucible_amd/csrc/common.hpp",
                  "crucible_amd/csrc/generic_attend.hpp", "include/crucible_attn.h")


def source_sha() -> str:
    """Hash of the decode kernel's sources and build flags: a profile summary applies to the
    kernel built from exactly these."""
    import hashlib

    from crucible_amd import _build

    h = hashlib.sha256()
    for name in DECODE_SOURCES:
        with open(os.path.join(ROOT, name), "rb") as f:
            h.update(name.encode() + b"\0" + f.read())
    flags = [_build.ARCH, *_build.HIPCC_FLAGS, *_build.EXTRA_FLAGS.get("attn_decode.hip", [])]
    h.update(b"flags\0" + "\0".join(flags).encode())
    return h.hexdigest()[:16]


def decode_kernel_name(gpu, batch, n_head, n_kv, max_seq, entry) -> str:
    """The kernel the library launches for this decode call (its own launch choices)."""
    import ctypes

    from crucible_amd import _lib

    buf = ctypes.create_string_buffer(128)
    _lib.check(gpu.lib.crucible_attention_decode_kernel_name(batch, n_head, n_kv, max_seq,
                                                             _lib.F16, entry, buf, 128))
    return buf.value.decode()


# ---------------------------------------------------------------- main

def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(a multi-GPU run would shard the attention path by sequence or KV head)",
              file=sys.stderr)
        sys.exit(2)
    import numpy as np  # noqa: F401
    import torch

    if args.phases:  # bind the stamped twin before anything loads the product library
        from crucible_amd import _build, _lib
        _lib.load(_build.STAMPS_LIB_PATH)
    from crucible_amd import workloads as W
    from crucible_amd.gpu import Gpu, tuning_state

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    gpu = Gpu(0)

    def log(msg):
        print(f"[bench] {msg}", file=sys.stderr, flush=True)

    log(f"{gpu.version()} on {torch.cuda.get_device_name(0)}")
    envelope_start = power_envelope()
    log(f"power envelope: {envelope_start}")
    if args.phases:
        fn = decode_phases if args.phases == "decode" else prefill_phases
        print(json.dumps(fn(gpu, dev, args, log)), flush=True)
        return
    b16 = DecodeBench(gpu, dev, batch=16, n_head=12, n_kv_head=args.kv_heads, n_layer=12,
                      n_pages=8192, max_seq=2048, rotations=7, seed=W.BASE_SEED + 2)
    log(f"config 3: {b16.rotations} rotations, lens of rotation 0: {b16.lens[0].tolist()}")
    step_graphs = b16.capture("fused")
    log("graphs captured")

    # headline: the whole step (12 fused append + decode launches), timed steps
    ms_per_step, ev_ms_per_step, step_bytes = b16.time_steps(step_graphs, args.steps,
                                                             args.warmup)
    envelope_headline = power_envelope()  # right after the timed steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"timed {args.steps} steps: {ms_per_step:.4f} ms/step (events {ev_ms_per_step:.4f}), "
        f"{value:.1f} GB/s")

    # dominant kernel: the fused decode kernel is the only kernel of the step, so its
    # average launch duration is the event-timed step over its 12 launches (graph replay:
    # each launch starts when the previous one ends, as in the rocprof trace)
    launch_us = ev_ms_per_step * 1e3 / b16.n_layer
    bytes_per_launch = step_bytes / b16.n_layer
    achieved = bytes_per_launch / (launch_us * 1e-6) / 1e9
    log(f"fused decode launch: {launch_us:.2f} us avg, {achieved:.1f} GB/s")
    kernel = decode_kernel_name(gpu, 16, 12, args.kv_heads, 2048, 1)
    copy_gbs = copy_bandwidth(dev)
    log(f"device copy: {copy_gbs:.1f} GB/s (read + write)")
    floor_us = launch_floor_us(dev)
    log(f"launch floor: {floor_us:.2f} us per launch of a one-element kernel in a graph")
    roofline = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": pmc_traffic(kernel),
                "kernel": kernel,
                "kernel_role": "append + split-K attention + combine, one launch per layer",
                "us_per_launch": round(launch_us, 3),
                "algorithmic_bytes_per_launch": int(bytes_per_launch),
                "copy_gbs": round(copy_gbs, 1),
                "frac_of_copy": round(achieved / copy_gbs, 4),
                "launch_floor_us": round(floor_us, 3),
                "source_sha": source_sha()}
    del step_graphs

    extras = {}
    groups = set() if args.no_extras else {g.strip() for g in args.extras.split(",")}
    if "decode" in groups:
        # the reference's three launches per layer, and attention alone, same batches
        for mode in ("separate", "decode"):
            graphs = b16.capture(mode)
            attn_only = (lambda r: b16.n_layer * b16.decode_bytes(r)) if mode == "decode" else None
            ms, ev, by = b16.time_steps(graphs, max(60, args.steps // 4), 10, attn_only)
            extras[f"step_{mode}"] = {"ms_per_step": round(ms, 5),
                                      "us_per_layer": round(ev * 1e3 / b16.n_layer, 3),
                                      "gbs": round(by / (ev * 1e-3) / 1e9, 2)}
            del graphs
        # config 2: batch 1, ctx 1024, 4096-page pool
        b1 = DecodeBench(gpu, dev, batch=1, n_head=12, n_kv_head=args.kv_heads, n_layer=12,
                         n_pages=4096, max_seq=1024, rotations=48, seed=W.BASE_SEED + 1,
                         fixed_lens=[1024])
        graphs = b1.capture("decode")
        ms, ev, _ = b1.time_steps(graphs, 96, 10)
        by1 = b1.decode_bytes(0)
        extras["decode_b1_ctx1024"] = {"us_per_launch": round(ev * 1e3 / 12, 3),
                                       "gbs": round(by1 / (ev * 1e-3 / 12) / 1e9, 2),
                                       "bytes_per_launch": int(by1)}
        if not args.no_cpu_baseline:
            reps, s_step, cores, model = cpu_decode(b1, 2.0)
            extras["decode_b1_ctx1024"]["cpu"] = {
                "us_per_layer": round(s_step * 1e6 / 12, 2), "cores": cores, "kind": "port",
                "cpu_model": model,
                "sample": f"median of {reps} 12-layer steps after 5 warmups, the GPU run's bytes"}
        del graphs, b1
        if args.kv_heads != 12:
            mha = DecodeBench(gpu, dev, batch=16, n_head=12, n_kv_head=12, n_layer=12,
                              n_pages=8192, max_seq=2048, rotations=7, seed=W.BASE_SEED + 2)
            graphs = mha.capture("fused")
            ms, ev, by = mha.time_steps(graphs, 60, 10)
            gbs = by / (ev * 1e-3) / 1e9
            extras["fused_b16_mha12"] = {"us_per_launch": round(ev * 1e3 / 12, 3),
                                         "gbs": round(gbs, 2),
                                         "frac": round(gbs / HBM_PEAK_GBS, 4),
                                         "bytes_per_launch": int(by / 12)}
            del graphs, mha
        torch.cuda.empty_cache()
    if "scale" in groups:
        # the same kernel and length distribution with more bytes per launch: where the
        # bandwidth goes once a launch is no longer latency-bound
        scale = {}
        for kv, batches in ((3, (32, 64, 128, 256)), (12, (32, 64))):
            for batch in batches:
                sb = DecodeBench(gpu, dev, batch=batch, n_head=12, n_kv_head=kv, n_layer=12,
                                 n_pages=batch * 3 * 140, max_seq=2048, rotations=3,
                                 seed=W.BASE_SEED + 2)
                graphs = sb.capture("fused")
                ms, ev, by = sb.time_steps(graphs, 60, 10)
                gbs = by / (ev * 1e-3) / 1e9
                scale[f"b{batch}_kv{kv}"] = {"us_per_launch": round(ev * 1e3 / 12, 2),
                                             "mb_per_launch": round(by / 12 / 1e6, 1),
                                             "gbs": round(gbs, 1),
                                             "frac": round(gbs / HBM_PEAK_GBS, 4)}
                del graphs, sb
                torch.cuda.empty_cache()
        extras["decode_scale"] = scale
    if "scale" in groups or "pscale" in groups:
        # prefill with longer sequences: the MFMA rate once a launch is compute-heavy
        pscale = {}
        for name, lens, nh, nkv in (("seq2048_12h", [2048], 12, 12), ("seq4096_12h", [4096], 12, 12),
                                    ("seq8192_12h", [8192], 12, 12),
                                    ("packed8x2048_16h4kv", [2048] * 8, 16, 4)):
            r = bench_prefill(gpu, dev, W.prefill_sequences(name, lens, nh, nkv), launches=10)
            pscale[name] = {k: r[k] for k in ("us_per_launch", "tflops", "frac_of_mfma_f16_peak",
                                              "p_operand", "gfx_clk_mhz",
                                              "frac_of_mfma_f16_peak_at_clock")}
            torch.cuda.empty_cache()
        extras["prefill_scale"] = pscale
    if "prefill" in groups:
        for key, cfg in (("prefill_config1", W.config1_prefill(n_kv_head=12)),
                         ("prefill_config1_gqa3", W.config1_prefill(n_kv_head=3)),
                         ("packed_config4", W.config4_packed())):
            inputs = {} if not args.no_cpu_baseline else None
            extras[key] = bench_prefill(gpu, dev, cfg, cpu_inputs=inputs)
            if inputs:
                extras[key]["cpu"] = cpu_prefill(cfg, inputs, 2.0)
        torch.cuda.empty_cache()
    if "e2e" in groups:
        extras["e2e_config5"] = bench_e2e(gpu)
    for k, v in extras.items():
        log(f"{k}: {v}")

    if args.copy_probe:
        src = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize(dev)
        log("copy probe: 5 x 256 MiB device copies")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(b16, args.cpu_seconds)
        log(f"cpu baseline: {cpu}")
        if extras:
            log("cpu beside the extras: " + str({k: v.get("cpu") for k, v in extras.items()
                                                 if isinstance(v, dict) and "cpu" in v}))

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "tuning": tuning_state(),
        "config": {"workload": "config3 paged decode b16, ctx U[64,2048], 12 layers, "
                               "append + attention per layer",
                   "batch": 16, "n_head": 12, "n_kv_head": args.kv_heads, "head_dim": 64,
                   "n_layer": 12, "page_tokens": 16, "pool_pages": 8192,
                   "rotations": b16.rotations, "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4)},
        "roofline": roofline,
        "envelope": {"start": envelope_start, "after_headline": envelope_headline,
                     "end": power_envelope()},
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

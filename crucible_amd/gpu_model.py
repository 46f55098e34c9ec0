"""Batched greedy decoding of a crucible-architecture decoder over this library.

The caller side of the attention path, after the reference's device model
(engine/src/gpu_model.rs): packed prefill of every prompt
(queue_prefill_transformer_impl, :3254-3580), then batched single-token decode steps
(queue_decode_batch, :1393-1605) captured once in a HIP graph and replayed, with the
greedy token chosen on the device (argmax_rows, :1585-1586).

Per layer the attention block is this library:
  * prefill: crucible_cache_store_packed_paged for K and V, then
    crucible_attention_prefill_tiled over {packed_start, chunk_len, 0, table} segments;
  * decode: crucible_attention_decode_paged_append (both row appends and the attention
    in one launch).
Projections, norms and the MLP follow the reference CPU arithmetic
(engine/src/model.rs:145-299, engine/src/ops.rs): RMSNorm with the mean of squares and
the scale in f64, half-split RoPE from f32 tables whose angles are computed in f64,
SwiGLU as g / (1 + exp(-g)) * u, pre-norm residual blocks, and a vocabulary projection
tied to the token embedding. Activations are f32, weights fp16, KV pages fp16.
Projections run either as the reference's matvec contract (ops.rs:17-32: f32 operands,
f64 accumulation, f32 result; `precision="reference"`) or as plain f32 GEMMs
(`precision="f32"`). In reference precision the decode step is this library's kernels
end to end: f64-MFMA projections with RMSNorm, residual and SwiGLU fused
(crucible_linear_f64acc, crucible_linear_swiglu_f64acc), RoPE of q and k fused with both
appends and the attention (crucible_attention_decode_qkv_paged_append), RMSNorm and the
vocabulary projection, then the device argmax. The prefill's projections are torch f64
GEMMs (the same contract) over the packed rows.

Paging is the reference allocator (crucible_amd.paged): every request reserves the
pages it needs through its last generated token up front (prefill.rs:160-172), so the
tables do not change while the decode graph replays.
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass

import numpy as np
import torch

from .gpu import Gpu
from .paged import PagePool, SequencePages, request_page_reservation, segments_from_cu_seqlens

PAGE_TOKENS = 16


@dataclass(frozen=True)
class ModelConfig:
    """The reference GPTConfig fields this path needs (model.py:47-99)."""
    n_layer: int = 12
    n_head: int = 12
    n_kv_head: int = 3
    n_embd: int = 768
    hidden: int = 2048          # SwiGLU width: round64(2 * 4 * n_embd / 3), model.py:222-229
    vocab_size: int = 50257
    block_size: int = 1024      # reference context capacity
    rope_theta: float = 10000.0
    norm_eps: float = 1e-6      # model.rs:20

    @property
    def head_dim(self) -> int:
        return self.n_embd // self.n_head

    @property
    def kv_dim(self) -> int:
        return self.n_kv_head * self.head_dim


PRESET_120M = ModelConfig()


def weight_names(cfg: ModelConfig) -> list[str]:
    names = ["tok_emb.weight"]
    for i in range(cfg.n_layer):
        p = f"blocks.{i}"
        names += [f"{p}.attn_norm.weight", f"{p}.attn.q_proj.weight", f"{p}.attn.k_proj.weight",
                  f"{p}.attn.v_proj.weight", f"{p}.attn.o_proj.weight", f"{p}.mlp_norm.weight",
                  f"{p}.mlp.gate_proj.weight", f"{p}.mlp.up_proj.weight",
                  f"{p}.mlp.down_proj.weight"]
    return names + ["final_norm.weight"]


def weight_shape(cfg: ModelConfig, name: str) -> tuple[int, ...]:
    d, kv, hid = cfg.n_embd, cfg.kv_dim, cfg.hidden
    if name == "tok_emb.weight":
        return (cfg.vocab_size, d)
    if name.endswith("norm.weight"):
        return (d,)
    tail = name.split(".", 2)[2]
    return {"attn.q_proj.weight": (d, d), "attn.k_proj.weight": (kv, d),
            "attn.v_proj.weight": (kv, d), "attn.o_proj.weight": (d, d),
            "mlp.gate_proj.weight": (hid, d), "mlp.up_proj.weight": (hid, d),
            "mlp.down_proj.weight": (d, hid)}[tail]


def random_weights(cfg: ModelConfig, seed: int, std: float = 0.02) -> dict[str, np.ndarray]:
    """Random-init weights of the BASELINE config-5 model: every matrix N(0, std) rounded
    to fp16 (numpy's seeded generator), norm weights 1 (RMSNorm's init, model.py:118)."""
    rng = np.random.default_rng(seed)
    out = {}
    for name in weight_names(cfg):
        shape = weight_shape(cfg, name)
        if name.endswith("norm.weight"):
            out[name] = np.ones(shape, np.float16)
        else:
            out[name] = (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(
                np.float16)
    return out


def rope_tables(head_dim: int, max_seq: int, theta: float):
    """ops.rs:99-115: angles in f64, tables stored as f32, [max_seq][head_dim / 2]."""
    half = head_dim // 2
    inv = np.power(float(theta), -(2.0 * np.arange(half, dtype=np.float64)) / head_dim)
    ang = np.arange(max_seq, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


class GpuModel:
    """Greedy generation for up to `max_batch` requests of at most `capacity` tokens."""

    def __init__(self, cfg: ModelConfig, weights: dict[str, np.ndarray], *, max_batch: int,
                 capacity: int, device=0, gpu: Gpu | None = None,
                 precision: str = "reference"):
        if cfg.head_dim != 64:
            raise ValueError("this build implements head_dim 64")
        if precision not in ("reference", "f32"):
            raise ValueError("precision is 'reference' (f64-accumulated projections) or 'f32'")
        torch.backends.cuda.matmul.allow_tf32 = False
        self.precision = precision
        self.cfg = cfg
        self.gpu = gpu or Gpu(device)
        self.dev = self.gpu.device
        self.max_batch = max_batch
        self.capacity = capacity
        self.table_stride = -(-capacity // PAGE_TOKENS)
        dev = self.dev

        def f32(name):
            return torch.from_numpy(np.ascontiguousarray(weights[name])).to(dev).float()

        def h16(name):  # projection weights stay fp16 on the device
            return torch.from_numpy(np.ascontiguousarray(weights[name])).to(dev).half()

        self.tok_emb = f32("tok_emb.weight")
        self.lm_head = h16("tok_emb.weight")  # tied (model.rs:288-297)
        self.layers = []
        for i in range(cfg.n_layer):
            p = f"blocks.{i}"
            # gate and up rows in one buffer, so the o projection can prefetch both as one
            # region
            wgu = torch.cat([h16(f"{p}.mlp.gate_proj.weight"),
                             h16(f"{p}.mlp.up_proj.weight")]).contiguous()
            self.layers.append({
                "attn_norm": f32(f"{p}.attn_norm.weight"),
                "wqkv": torch.cat([h16(f"{p}.attn.q_proj.weight"),
                                   h16(f"{p}.attn.k_proj.weight"),
                                   h16(f"{p}.attn.v_proj.weight")]).contiguous(),
                "wo": h16(f"{p}.attn.o_proj.weight"),
                "mlp_norm": f32(f"{p}.mlp_norm.weight"),
                "wgu": wgu,
                "wg": wgu[:cfg.hidden],
                "wu": wgu[cfg.hidden:],
                "wd": h16(f"{p}.mlp.down_proj.weight"),
            })
        self.final_norm = f32("final_norm.weight")
        cos, sin = rope_tables(cfg.head_dim, capacity, cfg.rope_theta)
        self.rope_cos = torch.from_numpy(cos).to(dev)
        self.rope_sin = torch.from_numpy(sin).to(dev)

        pages_per_req = self.table_stride
        self.n_pages = max_batch * pages_per_req + 1
        elems = self.n_pages * cfg.n_layer * PAGE_TOKENS * cfg.kv_dim
        self.k_pool = torch.zeros(elems, dtype=torch.float16, device=dev)
        self.v_pool = torch.zeros(elems, dtype=torch.float16, device=dev)
        self.page_pool = PagePool(self.n_pages, cfg.n_layer, cfg.kv_dim)
        self.workspace = self.gpu.workspace(max_batch, cfg.n_head, capacity)
        self._graph = None
        self._graph_batch = None

    # ------------------------------------------------------------------ glue ops
    def _linear(self, x, w):
        """x [rows, in] f32 times the fp16 w [out, in]^T: f64 products and sums rounded
        once to f32 (reference precision) or an f32 GEMM."""
        if self.precision == "f32":
            return x @ w.float().t()
        return (x.double() @ w.double().t()).float()

    def _rmsnorm(self, x, w):
        """ops.rs rmsnorm: scale = 1 / sqrt(mean(x^2) + eps) in f64, out = f32(x * scale) * w."""
        xd = x.double()
        scale = 1.0 / torch.sqrt(xd.pow(2).mean(-1, keepdim=True) + float(np.float32(self.cfg.norm_eps)))
        return (xd * scale).float() * w

    def _rope(self, x, cos, sin, n_heads):
        """ops.rs RopeTable::apply: element i pairs with i + 32; lo*c - hi*s, lo*s + hi*c."""
        rows = x.shape[0]
        xv = x.view(rows, n_heads, 64)
        lo, hi = xv[..., :32], xv[..., 32:]
        c = cos.unsqueeze(1)
        s = sin.unsqueeze(1)
        return torch.cat([lo * c - hi * s, lo * s + hi * c], dim=-1).reshape(rows, n_heads * 64)

    def _mlp(self, x, layer):
        h = self._rmsnorm(x, layer["mlp_norm"])
        g = self._linear(h, layer["wg"])
        u = self._linear(h, layer["wu"])
        a = g / (1.0 + torch.exp(-g)) * u
        return x + self._linear(a, layer["wd"])

    def _qkv(self, x, layer, cos, sin):
        cfg = self.cfg
        h = self._rmsnorm(x, layer["attn_norm"])
        qkv = self._linear(h, layer["wqkv"])
        d, kv = cfg.n_embd, cfg.kv_dim
        q = self._rope(qkv[:, :d], cos, sin, cfg.n_head)
        k = self._rope(qkv[:, d:d + kv], cos, sin, cfg.n_kv_head)
        v = qkv[:, d + kv:].contiguous()
        return q, k, v

    def _logits(self, x):
        return self._linear(self._rmsnorm(x, self.final_norm), self.lm_head)

    # ------------------------------------------------------------------ requests
    def _admit(self, prompts, n_new):
        seqs, tables = [], np.zeros((len(prompts), self.table_stride), np.int32)
        for b, p in enumerate(prompts):
            need = request_page_reservation(len(p), n_new, self.capacity)
            if need > self.table_stride:
                raise ValueError(f"request {b} needs {need} pages > table stride")
            s = SequencePages()
            s.grow(self.page_pool, need * PAGE_TOKENS)
            tables[b] = s.table_padded(self.table_stride)
            seqs.append(s)
        return seqs, tables

    def _release(self, seqs):
        for s in seqs:
            s.release(self.page_pool)

    # ------------------------------------------------------------------ prefill
    @torch.no_grad()
    def prefill(self, prompts, d_tables):
        """Packed prefill of every prompt; returns the device int32 first token per request
        and the final-row logits."""
        cfg, gpu, dev = self.cfg, self.gpu, self.dev
        lens = np.array([len(p) for p in prompts], np.int32)
        cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        rows = int(cu[-1])
        seg, max_chunk = segments_from_cu_seqlens(cu)
        owners = np.repeat(np.arange(len(prompts), dtype=np.int32), lens)
        positions = np.concatenate([np.arange(n, dtype=np.int32) for n in lens])
        d_seg = torch.from_numpy(np.ascontiguousarray(seg)).to(dev)
        d_own = torch.from_numpy(owners).to(dev)
        d_pos = torch.from_numpy(positions).to(dev)
        tok = torch.from_numpy(np.concatenate([np.asarray(p, np.int64) for p in prompts])).to(dev)
        x = self.tok_emb.index_select(0, tok)
        if self.precision == "reference":
            # this library's projections (f64-accumulated, norms, RoPE, SwiGLU and the
            # residual adds fused as in the decode step) over every prompt row
            return self._prefill_native(prompts, x, cu, d_tables, d_seg, d_own, d_pos, max_chunk)
        cos = self.rope_cos.index_select(0, d_pos)
        sin = self.rope_sin.index_select(0, d_pos)
        attn = torch.empty((rows, cfg.n_embd), dtype=torch.float32, device=dev)
        for layer_i, layer in enumerate(self.layers):
            q, k, v = self._qkv(x, layer, cos, sin)
            for src, pool, kind in ((k, self.k_pool, "k"), (v, self.v_pool, "v")):
                gpu.cache_store_packed_paged(src, pool, d_tables, d_own, d_pos, rows, cfg.kv_dim,
                                             self.table_stride, cfg.n_layer, layer_i, kind=kind)
            gpu.attention_prefill_tiled(q, self.k_pool, self.v_pool, None, None, attn, d_tables,
                                        d_seg, len(prompts), max_chunk, self.table_stride,
                                        cfg.n_head, cfg.n_kv_head, 64, cfg.n_layer, layer_i,
                                        cfg.kv_dim)
            x = x + self._linear(attn, layer["wo"])
            x = self._mlp(x, layer)
        last = torch.from_numpy(cu[1:] - 1).long().to(dev)
        logits = self._logits(x.index_select(0, last)).contiguous()
        first = torch.empty(len(prompts), dtype=torch.int32, device=dev)
        gpu.argmax_rows(logits, first, len(prompts), cfg.vocab_size)
        return first, logits

    def _prefill_native(self, prompts, x, cu, d_tables, d_seg, d_own, d_pos, max_chunk):
        """The packed prefill as this library's kernels (the reference CPU arithmetic of
        model.rs:145-299 over all prompt rows at once): per layer the q/k/v projection with
        the attention RMSNorm fused, RoPE and the q/k/v split, both packed appends, the tiled
        prefill attention, the o projection with the residual add, the gate/up projection
        with the MLP norm and SwiGLU, and the down projection with the residual add; then the
        vocabulary projection of each prompt's last row with the final norm fused."""
        cfg, gpu, dev = self.cfg, self.gpu, self.dev
        rows = x.shape[0]
        eps = float(np.float32(cfg.norm_eps))
        d, kv = cfg.n_embd, cfg.kv_dim
        qkv = torch.empty((rows, d + 2 * kv), dtype=torch.float32, device=dev)
        q = torch.empty((rows, d), dtype=torch.float32, device=dev)
        k = torch.empty((rows, kv), dtype=torch.float32, device=dev)
        v = torch.empty((rows, kv), dtype=torch.float32, device=dev)
        attn = torch.empty((rows, d), dtype=torch.float32, device=dev)
        act = torch.empty((rows, cfg.hidden), dtype=torch.float32, device=dev)
        x = x.contiguous()
        for layer_i, layer in enumerate(self.layers):
            gpu.linear_f64acc(x, layer["wqkv"], qkv, norm_w=layer["attn_norm"], eps=eps)
            gpu.rope_split_qkv(qkv, q, k, v, self.rope_cos, self.rope_sin, d_pos, cfg.n_head,
                               cfg.n_kv_head)
            for src, pool, kind in ((k, self.k_pool, "k"), (v, self.v_pool, "v")):
                gpu.cache_store_packed_paged(src, pool, d_tables, d_own, d_pos, rows, kv,
                                             self.table_stride, cfg.n_layer, layer_i, kind=kind)
            gpu.attention_prefill_tiled(q, self.k_pool, self.v_pool, None, None, attn, d_tables,
                                        d_seg, len(prompts), max_chunk, self.table_stride,
                                        cfg.n_head, cfg.n_kv_head, 64, cfg.n_layer, layer_i, kv)
            gpu.linear_f64acc(attn, layer["wo"], x, resid=x)
            gpu.linear_swiglu_f64acc(x, layer["wg"], layer["wu"], act, norm_w=layer["mlp_norm"],
                                     eps=eps)
            gpu.linear_f64acc(act, layer["wd"], x, resid=x)
        last = torch.from_numpy(cu[1:] - 1).long().to(dev)
        xl = x.index_select(0, last).contiguous()
        logits = torch.empty((len(prompts), cfg.vocab_size), dtype=torch.float32, device=dev)
        gpu.linear_f64acc(xl, self.lm_head, logits, norm_w=self.final_norm, eps=eps)
        first = torch.empty(len(prompts), dtype=torch.int32, device=dev)
        gpu.argmax_rows(logits, first, len(prompts), cfg.vocab_size)
        return first, logits

    @torch.no_grad()
    def prefill_logits(self, prompts) -> np.ndarray:
        """Logits of each prompt's last position after a packed prefill (host f32)."""
        seqs, tables = self._admit(prompts, 1)
        try:
            _, logits = self.prefill(prompts, torch.from_numpy(tables).to(self.dev))
            return logits.cpu().numpy()
        finally:
            self._release(seqs)

    # ------------------------------------------------------------------ decode
    def _decode_step(self, st):
        """One batched decode step on the static buffers in `st` (graph-capturable)."""
        if self.precision == "reference":
            self._decode_step_native(st)
        else:
            self._decode_step_torch(st)
            self._advance(st)

    def _decode_step_native(self, st):
        """The step as this library's kernels (reference arithmetic), 5 launches a layer,
        then the vocabulary projection (with the final norm) and the greedy tail. st["x"]
        enters as the embedding of the token fed (the previous step's greedy tail, or the
        caller, wrote it) and leaves as the next one's."""
        cfg, gpu = self.cfg, self.gpu
        b = st["batch"]
        eps = float(np.float32(cfg.norm_eps))
        x = st["x"]
        # Each projection fetches the next one's weights into the last-level cache while it
        # runs (the step streams more than that cache holds, so they would arrive cold).
        for layer_i, layer in enumerate(self.layers):
            nxt = self.layers[layer_i + 1]["wqkv"] if layer_i + 1 < cfg.n_layer else None
            gpu.linear_f64acc(x, layer["wqkv"], st["qkv"], norm_w=layer["attn_norm"], eps=eps,
                              prefetch=layer["wo"])
            # RoPE of q and k, both appends and attention: one launch on the fused rows
            gpu.attention_decode_qkv_paged_append(st["qkv"], self.rope_cos, self.rope_sin,
                                                  self.k_pool, self.v_pool, st["attn"],
                                                  st["tables"], st["positions"], st["lens"], b,
                                                  cfg.n_head, cfg.n_kv_head, 64,
                                                  self.table_stride, cfg.n_layer, layer_i,
                                                  cfg.kv_dim, self.capacity,
                                                  workspace=self.workspace)
            gpu.linear_f64acc(st["attn"], layer["wo"], x, resid=x, prefetch=layer["wgu"])
            gpu.linear_swiglu_f64acc(x, layer["wg"], layer["wu"], st["act"],
                                     norm_w=layer["mlp_norm"], eps=eps, prefetch=layer["wd"])
            gpu.linear_f64acc(st["act"], layer["wd"], x, resid=x, prefetch=nxt)
        gpu.linear_f64acc(x, self.lm_head, st["logits"], norm_w=self.final_norm, eps=eps)
        gpu.greedy_advance(st["logits"], self.tok_emb, x, st["tokens"], st["history"],
                           st["step"], st["positions"], st["lens"], st["done"])

    def _decode_step_torch(self, st):
        cfg, gpu = self.cfg, self.gpu
        b = st["batch"]
        cos = self.rope_cos.index_select(0, st["positions"])
        sin = self.rope_sin.index_select(0, st["positions"])
        x = self.tok_emb.index_select(0, st["tokens"])
        for layer_i, layer in enumerate(self.layers):
            q, k, v = self._qkv(x, layer, cos, sin)
            gpu.attention_decode_paged_append(q, k, v, self.k_pool, self.v_pool, st["attn"],
                                              st["tables"], st["positions"], st["lens"], b,
                                              cfg.n_head, cfg.n_kv_head, 64, self.table_stride,
                                              cfg.n_layer, layer_i, cfg.kv_dim, self.capacity,
                                              workspace=self.workspace)
            x = x + self._linear(st["attn"], layer["wo"])
            x = self._mlp(x, layer)
        st["logits"].copy_(self._logits(x))

    def _advance(self, st):
        """Greedy token, history, and the next step's position and length."""
        b = st["batch"]
        self.gpu.argmax_rows(st["logits"], st["tokens"], b, self.cfg.vocab_size)
        st["history"].index_copy_(0, st["step"], st["tokens"].view(1, b))
        st["positions"].add_(1)
        st["lens"].add_(1)
        st["step"].add_(1)

    @torch.no_grad()
    def generate(self, prompts, n_new: int, *, graph: bool = True, timing: dict | None = None):
        """Greedy-generate n_new tokens per prompt; returns int32 [batch, n_new] (host).

        The first token comes from the prefill logits; each decode step consumes the
        previous token at the next position and produces one more."""
        cfg, dev = self.cfg, self.dev
        batch = len(prompts)
        if batch > self.max_batch:
            raise ValueError("batch exceeds max_batch")
        if any(len(p) == 0 for p in prompts):
            raise ValueError("empty prompt")
        if max(len(p) for p in prompts) + n_new - 1 > self.capacity:
            raise ValueError("request exceeds capacity")
        seqs, tables = self._admit(prompts, n_new)
        try:
            d_tables = torch.from_numpy(tables).to(dev)
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
            ev[0].record()
            first, _ = self.prefill(prompts, d_tables)
            ev[1].record()
            lens = np.array([len(p) for p in prompts], np.int32)
            st = {
                "batch": batch,
                "tables": d_tables,
                "tokens": first.clone(),
                "positions": torch.from_numpy(lens).to(dev),       # position of the token fed
                "lens": torch.from_numpy(lens + 1).to(dev),        # keys visible after append
                "attn": torch.empty((batch, cfg.n_embd), dtype=torch.float32, device=dev),
                "x": torch.empty((batch, cfg.n_embd), dtype=torch.float32, device=dev),
                "qkv": torch.empty((batch, cfg.n_embd + 2 * cfg.kv_dim), dtype=torch.float32,
                                   device=dev),
                "act": torch.empty((batch, cfg.hidden), dtype=torch.float32, device=dev),
                "logits": torch.empty((batch, cfg.vocab_size), dtype=torch.float32, device=dev),
                "history": torch.zeros((max(n_new - 1, 1), batch), dtype=torch.int32, device=dev),
                "step": torch.zeros(1, dtype=torch.long, device=dev),
                "done": torch.zeros(1, dtype=torch.int32, device=dev),
            }
            if self.precision == "reference":  # the first step's input row
                torch.index_select(self.tok_emb, 0, st["tokens"], out=st["x"])
            steps = n_new - 1
            capture_s = 0.0
            if steps > 0 and graph:
                t0 = time.perf_counter()
                g = self._capture(st)  # once per call here; once per process in a server
                capture_s = time.perf_counter() - t0
                ev[2].record()  # the decode loop: the replays only
                for _ in range(steps):
                    g.replay()
            else:
                ev[2].record()
                for _ in range(steps):
                    self._decode_step(st)
            ev[3].record()
            torch.cuda.synchronize(dev)
            if timing is not None:
                timing["prefill_ms"] = ev[0].elapsed_time(ev[1])
                timing["decode_ms"] = ev[2].elapsed_time(ev[3])
                timing["decode_steps"] = steps
                timing["capture_ms"] = capture_s * 1e3
            out = np.empty((batch, n_new), np.int32)
            out[:, 0] = first.cpu().numpy()
            if steps > 0:
                out[:, 1:] = st["history"][:steps].cpu().numpy().T
            return out
        finally:
            self._release(seqs)

    def _capture(self, st):
        """Capture one decode step. Warm-up runs on a side stream first (torch's rule);
        they advance the step state, so it is saved and restored around them."""
        saved = {k: v.clone() for k, v in st.items() if isinstance(v, torch.Tensor)}
        side = torch.cuda.Stream(self.dev)
        side.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(side):
            self._decode_step(st)
        torch.cuda.current_stream(self.dev).wait_stream(side)
        torch.cuda.synchronize(self.dev)
        for k, v in saved.items():
            st[k].copy_(v)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._decode_step(st)
        # capture does not run the step: restore the state the replay starts from
        for k, v in saved.items():
            st[k].copy_(v)
        torch.cuda.synchronize(self.dev)
        return g


def seeded_prompts(seed: int, batch: int, lo: int, hi: int, vocab: int) -> list[list[int]]:
    """BASELINE config 5 prompts: lengths U[lo, hi], token ids U[0, vocab) (numpy seeded)."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=batch)
    return [rng.integers(0, vocab, size=int(n)).tolist() for n in lens]


__all__ = ["ModelConfig", "PRESET_120M", "GpuModel", "random_weights", "rope_tables",
           "seeded_prompts", "weight_names", "weight_shape", "math"]

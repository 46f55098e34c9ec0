"""CPU oracle of the end-to-end greedy decode -- TEST INFRASTRUCTURE.

Only tests/ may use it, as the checker of crucible_amd.gpu_model. It restates the
reference CPU forward pass, engine/src/model.rs:145-299 (Model::forward_cached), with the
reference's helpers from engine/src/ops.rs:
  * matvec (:17-32): dot products accumulated in f64, rounded to f32 -- here numpy f64
    matrix products of the f32 operands (row order independent, so several positions
    or requests are processed together without changing any value);
  * rmsnorm (:37-50): sum of squares and the scale in f64, out = f32(x * scale) * w;
  * RopeTable (:94-136): f32 tables from f64 angles, half-split rotation in f32;
  * attention (model.rs:210-235 with ops.rs:67-80): reference-order f32 scores, softmax
    with an f64 normaliser, f32 P.V -- oracle.c's attend_one_ref_f32;
  * silu (:84-86) and the tied vocabulary projection (model.rs:288-297);
  * greedy selection: sampling.rs:141-150 (oracle.c orc_argmax).
The one change is the storage contract of the paged fp16 KV cache: K (after RoPE) and V
are rounded to fp16 (RNE) when they are written, as the GPU pools hold them. With
kv_fp16=False the cache keeps f32 values, which is the reference's own f32 cache
(engine/src/cache.rs:16-105); comparing the two measures what the storage change alone does
to greedy tokens (oracle/kv_storage_report.py).

Prompts are processed layer by layer over all their positions at once, which performs
exactly the per-position arithmetic of the reference's token-major loop (a position at
layer l reads only layer-l keys of itself and earlier positions).
"""
from __future__ import annotations

import numpy as np

from . import attention_dense, f16_bits_to_f32, f32_to_f16_bits, argmax


class OracleModel:
    def __init__(self, cfg, weights: dict[str, np.ndarray], kv_fp16: bool = True):
        self.cfg = cfg
        self.kv_fp16 = kv_fp16
        f64 = lambda n: weights[n].astype(np.float64)  # noqa: E731
        f32 = lambda n: weights[n].astype(np.float32)  # noqa: E731
        self.tok_emb32 = f32("tok_emb.weight")
        self.tok_emb64 = self.tok_emb32.astype(np.float64)
        self.layers = []
        for i in range(cfg.n_layer):
            p = f"blocks.{i}"
            self.layers.append({
                "attn_norm": f32(f"{p}.attn_norm.weight"),
                "wq": f64(f"{p}.attn.q_proj.weight"), "wk": f64(f"{p}.attn.k_proj.weight"),
                "wv": f64(f"{p}.attn.v_proj.weight"), "wo": f64(f"{p}.attn.o_proj.weight"),
                "mlp_norm": f32(f"{p}.mlp_norm.weight"),
                "wg": f64(f"{p}.mlp.gate_proj.weight"), "wu": f64(f"{p}.mlp.up_proj.weight"),
                "wd": f64(f"{p}.mlp.down_proj.weight"),
            })
        self.final_norm = f32("final_norm.weight")
        half = cfg.head_dim // 2
        inv = np.power(float(cfg.rope_theta), -(2.0 * np.arange(half)) / cfg.head_dim)
        ang = np.arange(cfg.block_size + 4096, dtype=np.float64)[:, None] * inv[None, :]
        self.cos = np.cos(ang).astype(np.float32)
        self.sin = np.sin(ang).astype(np.float32)

    # ---------------------------------------------------------------- ops
    @staticmethod
    def matvec(w64, x32):
        """ops.rs matvec over rows of x: f64 accumulation, f32 result."""
        return (x32.astype(np.float64) @ w64.T).astype(np.float32)

    def rmsnorm(self, x, w):
        xd = x.astype(np.float64)
        scale = 1.0 / np.sqrt((xd * xd).sum(-1, keepdims=True) / x.shape[-1]
                              + float(np.float32(self.cfg.norm_eps)))
        return (xd * scale).astype(np.float32) * w

    def rope(self, x, positions, n_heads):
        xv = x.reshape(x.shape[0], n_heads, self.cfg.head_dim)
        half = self.cfg.head_dim // 2
        c = self.cos[positions][:, None, :]
        s = self.sin[positions][:, None, :]
        lo, hi = xv[..., :half], xv[..., half:]
        out = np.concatenate([lo * c - hi * s, lo * s + hi * c], axis=-1)
        return out.reshape(x.shape).astype(np.float32)

    @staticmethod
    def silu_mul(g, u):
        return (g / (np.float32(1.0) + np.exp(-g))) * u

    # ---------------------------------------------------------------- model
    def _forward_rows(self, x, positions, owners, caches):
        """Run every layer over rows (positions[i] of request owners[i]) whose earlier
        positions are already cached; append their K/V; return the final hidden rows."""
        cfg = self.cfg
        for li, L in enumerate(self.layers):
            h = self.rmsnorm(x, L["attn_norm"])
            q = self.rope(self.matvec(L["wq"], h), positions, cfg.n_head)
            k = self.rope(self.matvec(L["wk"], h), positions, cfg.n_kv_head)
            v = self.matvec(L["wv"], h)
            if self.kv_fp16:  # paged fp16 storage contract
                k = f16_bits_to_f32(f32_to_f16_bits(k))
                v = f16_bits_to_f32(f32_to_f16_bits(v))
            attn = np.zeros_like(q)
            for b in np.unique(owners):
                sel = np.nonzero(owners == b)[0]
                kc, vc = caches[b][li]
                for i in sel:  # write this position's K/V
                    kc[positions[i]] = k[i]
                    vc[positions[i]] = v[i]
                n_keys = int(positions[sel].max()) + 1
                attn[sel] = attention_dense(q[sel], kc[:n_keys], vc[:n_keys],
                                            (positions[sel] + 1).astype(np.int32), cfg.n_head,
                                            cfg.n_kv_head, cfg.head_dim, precise=False)
            x = x + self.matvec(L["wo"], attn)
            h = self.rmsnorm(x, L["mlp_norm"])
            a = self.silu_mul(self.matvec(L["wg"], h), self.matvec(L["wu"], h))
            x = x + self.matvec(L["wd"], a)
        return x

    def logits(self, x):
        return self.matvec(self.tok_emb64, self.rmsnorm(x, self.final_norm))

    def generate(self, prompts, n_new: int, record_logits: bool = False):
        """Greedy tokens [batch, n_new] and, if asked, every step's logits."""
        cfg = self.cfg
        batch = len(prompts)
        cap = max(len(p) for p in prompts) + n_new
        caches = [[(np.zeros((cap, cfg.kv_dim), np.float32), np.zeros((cap, cfg.kv_dim), np.float32))
                   for _ in range(cfg.n_layer)] for _ in range(batch)]
        lens = np.array([len(p) for p in prompts])
        tokens = np.concatenate([np.asarray(p, np.int64) for p in prompts])
        positions = np.concatenate([np.arange(n) for n in lens])
        owners = np.repeat(np.arange(batch), lens)
        x = self._forward_rows(self.tok_emb32[tokens], positions, owners, caches)
        last = np.cumsum(lens) - 1
        logit_rows = self.logits(x[last])
        out = np.zeros((batch, n_new), np.int32)
        kept = [logit_rows] if record_logits else None
        out[:, 0] = [argmax(r) for r in logit_rows]
        pos = lens.copy()
        for step in range(1, n_new):
            x = self._forward_rows(self.tok_emb32[out[:, step - 1]], pos.copy(),
                                   np.arange(batch), caches)
            logit_rows = self.logits(x)
            if record_logits:
                kept.append(logit_rows)
            out[:, step] = [argmax(r) for r in logit_rows]
            pos += 1
        return (out, kept) if record_logits else out


def top2_gap(row: np.ndarray) -> float:
    """Logit distance between the best and the second-best token of one row."""
    top = np.partition(row.astype(np.float64), -2)[-2:]
    return float(top[1] - top[0])

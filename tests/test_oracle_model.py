"""Pins the end-to-end model oracle (oracle/model.py) on the CPU.

Against an independent float64 torch forward of the same architecture written the way
the reference's Python model writes it (model.py:139-145 apply_rope on chunks,
:185-213 causal SDPA with repeat_interleave for GQA, :222-246 SwiGLU, :103-121 RMSNorm,
:288-289 tied head), with the same fp16 K/V storage contract. The oracle's f32
reference-order arithmetic must agree with it to f32 accuracy, its greedy tokens must
follow the float64 argmax wherever the top-2 gap is not tiny, and incremental decoding
must equal a full forward over the generated prefix (the reference's cached == uncached
rule, model.rs:127-133).
"""
import numpy as np
import torch
import torch.nn.functional as F

from crucible_amd.gpu_model import ModelConfig, random_weights
from oracle.model import OracleModel, top2_gap

CFG = ModelConfig(n_layer=2, n_head=4, n_kv_head=2, n_embd=256, hidden=704, vocab_size=997,
                  block_size=256)


def _torch_forward(cfg, w, tokens):
    """Full causal forward of one sequence in float64; logits of every position."""
    d = torch.float64
    W = {k: torch.from_numpy(v.astype(np.float64)) for k, v in w.items()}
    T, hd, H, KV = len(tokens), cfg.head_dim, cfg.n_head, cfg.n_kv_head
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, hd, 2, dtype=d) / hd))
    freqs = torch.outer(torch.arange(T, dtype=d), inv)
    cos, sin = freqs.cos().float().double(), freqs.sin().float().double()

    def rope(x):  # x [1, heads, T, hd]
        x1, x2 = x.chunk(2, dim=-1)
        c, s = cos.view(1, 1, T, -1), sin.view(1, 1, T, -1)
        return torch.cat([x1 * c - x2 * s, x1 * s + x2 * c], dim=-1)

    def rms(x, g):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * g

    x = W["tok_emb.weight"][torch.tensor(tokens)].unsqueeze(0)
    for i in range(cfg.n_layer):
        p = f"blocks.{i}"
        h = rms(x, W[f"{p}.attn_norm.weight"])
        q = (h @ W[f"{p}.attn.q_proj.weight"].T).view(1, T, H, hd).transpose(1, 2)
        k = (h @ W[f"{p}.attn.k_proj.weight"].T).view(1, T, KV, hd).transpose(1, 2)
        v = (h @ W[f"{p}.attn.v_proj.weight"].T).view(1, T, KV, hd).transpose(1, 2)
        q, k = rope(q), rope(k)
        k, v = k.half().double(), v.half().double()      # paged fp16 storage contract
        k = k.repeat_interleave(H // KV, dim=1)
        v = v.repeat_interleave(H // KV, dim=1)
        y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        x = x + y.transpose(1, 2).reshape(1, T, -1) @ W[f"{p}.attn.o_proj.weight"].T
        h = rms(x, W[f"{p}.mlp_norm.weight"])
        g = h @ W[f"{p}.mlp.gate_proj.weight"].T
        u = h @ W[f"{p}.mlp.up_proj.weight"].T
        x = x + (F.silu(g) * u) @ W[f"{p}.mlp.down_proj.weight"].T
    return (rms(x, W["final_norm.weight"]) @ W["tok_emb.weight"].T)[0].numpy()


def test_oracle_logits_match_float64_torch_model():
    w = random_weights(CFG, seed=11, std=0.05)
    model = OracleModel(CFG, w)
    rng = np.random.default_rng(3)
    prompts = [rng.integers(0, CFG.vocab_size, size=n).tolist() for n in (1, 17, 40)]
    toks, logits = model.generate(prompts, 6, record_logits=True)
    for b, p in enumerate(prompts):
        full = list(p) + toks[b, :-1].tolist()
        ref = _torch_forward(CFG, w, full)                 # [T, vocab]
        for step in range(6):
            want = ref[len(p) - 1 + step]
            got = logits[step][b]
            np.testing.assert_allclose(got, want, rtol=2e-4, atol=2e-4)
            if top2_gap(want) > 1e-3:
                assert toks[b, step] == int(np.argmax(want))


def test_incremental_decode_equals_full_prefix_forward():
    """Generating token by token must give the logits a prefill of the whole prefix gives."""
    w = random_weights(CFG, seed=12, std=0.05)
    model = OracleModel(CFG, w)
    prompt = list(range(5, 30))
    toks, logits = model.generate([prompt], 4, record_logits=True)
    prefix = prompt + toks[0, :3].tolist()
    _, again = model.generate([prefix], 1, record_logits=True)
    np.testing.assert_array_equal(again[0][0], logits[3][0])

"""What the fp16 KV storage alone does to greedy decoding -- TEST INFRASTRUCTURE (CPU only).

Runs BASELINE config 5 (random-init 120m preset, 16 prompts of U[64, 512] seeded ids, 256
greedy tokens) through the CPU oracle twice: with the fp16 KV cache this build's pools hold
(the tokens the GPU path reproduces exactly, tests/test_gpu_e2e.py) and with the reference's
f32 cache (engine/src/cache.rs:16-105, kv_fp16=False). For every request it reports the
first generated token where the two differ and the top-2 logit gap of the f32-cache run at
that step (the reference reports the same quantity for its own divergences,
README.md:1205-1221); a gap near zero means the reference itself was at a near-tie there.

    python -m oracle.kv_storage_report [--tokens 256] [--requests 16]
"""
from __future__ import annotations

import argparse
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def compare(cfg, weights, prompts, n_new):
    """(tokens fp16-KV, tokens f32-KV, list of (request, step, gap, tok16, tok32))."""
    from oracle.model import OracleModel, top2_gap

    t16, _ = OracleModel(cfg, weights, kv_fp16=True).generate(prompts, n_new, record_logits=True)
    t32, logits32 = OracleModel(cfg, weights, kv_fp16=False).generate(prompts, n_new,
                                                                      record_logits=True)
    rows = []
    for b in range(len(prompts)):
        diff = np.nonzero(t16[b] != t32[b])[0]
        if diff.size:
            s = int(diff[0])
            rows.append((b, s, top2_gap(logits32[s][b]), int(t16[b, s]), int(t32[b, s])))
    return t16, t32, rows


def main():
    from crucible_amd.gpu_model import PRESET_120M, random_weights, seeded_prompts

    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--tokens", type=int, default=256)
    ap.add_argument("--requests", type=int, default=16)
    args = ap.parse_args()
    cfg = PRESET_120M
    seed = 20260908 + 4
    w = random_weights(cfg, seed=seed)
    prompts = seeded_prompts(seed, 16, 64, 512, cfg.vocab_size)[:args.requests]
    t0 = time.time()
    t16, t32, rows = compare(cfg, w, prompts, args.tokens)
    print(f"config 5, {len(prompts)} requests x {args.tokens} tokens, "
          f"{time.time() - t0:.0f} s on the CPU")
    same = len(prompts) - len(rows)
    print(f"{same} of {len(prompts)} requests token-identical between the fp16 and f32 KV caches")
    for b, s, gap, a16, a32 in rows:
        print(f"request {b} (prompt {len(prompts[b])} tokens): first difference at generated "
              f"token {s}: fp16 cache {a16}, f32 cache {a32}; f32-cache top-2 gap {gap:.3e}; "
              f"{int((t16[b] == t32[b]).sum())} of {args.tokens} tokens equal")


if __name__ == "__main__":
    main()

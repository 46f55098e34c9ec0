"""End-to-end greedy decode on the GPU against the CPU model oracle.

The GPU side is crucible_amd.gpu_model (packed prefill + graph-replayed batched decode
through this library's append, attention and argmax); the oracle is oracle/model.py,
the reference CPU forward (engine/src/model.rs) with the fp16 KV storage contract. The
bar is token identity; at a divergence the message reports the oracle's top-2 logit gap
at that step (the reference reports the same quantity, README.md:1205-1221).
"""
import numpy as np
import pytest
import torch

from crucible_amd.gpu_model import (PRESET_120M, GpuModel, ModelConfig, random_weights,
                                    seeded_prompts)
from oracle.model import OracleModel, top2_gap

pytestmark = pytest.mark.gpu

SMALL = ModelConfig(n_layer=2, n_head=4, n_kv_head=2, n_embd=256, hidden=704, vocab_size=997,
                    block_size=256)


def _compare(cfg, w, prompts, got, n_new, first_logits=None):
    want, logits = OracleModel(cfg, w).generate(prompts, n_new, record_logits=True)
    if first_logits is not None:
        d = np.abs(first_logits - logits[0]).max()
        print(f"max |logit| difference after prefill: {d:.3e}", flush=True)
    report = []
    for b in range(len(prompts)):
        diff = np.nonzero(got[b] != want[b])[0]
        if diff.size:
            s = int(diff[0])
            report.append(f"request {b} (prompt {len(prompts[b])} tokens) diverges at generated "
                          f"token {s}: gpu {got[b, s]} oracle {want[b, s]}, oracle top-2 gap "
                          f"{top2_gap(logits[s][b]):.3e}")
    print(f"{len(prompts) - len(report)} of {len(prompts)} requests token-identical over "
          f"{n_new} tokens", flush=True)
    if report:
        pytest.fail("\n".join(report))
    return want


def test_small_model_greedy_matches_oracle_and_graph_equals_eager(gpu, dev):
    w = random_weights(SMALL, seed=21, std=0.05)
    prompts = seeded_prompts(22, 5, 1, 60, SMALL.vocab_size)
    model = GpuModel(SMALL, w, max_batch=8, capacity=128, gpu=gpu)
    eager = model.generate(prompts, 24, graph=False)
    graph = model.generate(prompts, 24, graph=True)
    assert np.array_equal(eager, graph), "graph replay differs from eager execution"
    _compare(SMALL, w, prompts, graph, 24)
    # a second batch reuses the freed pages and the captured workspace
    again = model.generate(prompts[::-1], 24)
    assert np.array_equal(again, graph[::-1])


@pytest.mark.timeout(1200)
def test_config5_greedy_b16_256_tokens_token_identical(gpu, dev):
    """random-init 120m preset (12 layers, 12/3 heads, vocab 50257),
    fp16 weights N(0, 0.02), 16 prompts of U[64, 512] random ids, 256 greedy tokens each."""
    cfg = PRESET_120M
    w = random_weights(cfg, seed=20260908 + 4)
    prompts = seeded_prompts(20260908 + 4, 16, 64, 512, cfg.vocab_size)
    model = GpuModel(cfg, w, max_batch=16, capacity=1024, gpu=gpu)
    timing = {}
    got = model.generate(prompts, 256, timing=timing)
    first = model.prefill_logits(prompts)
    print(f"config5: prefill {timing['prefill_ms']:.2f} ms, decode {timing['decode_ms']:.2f} ms "
          f"for {timing['decode_steps']} steps "
          f"({16 * timing['decode_steps'] / timing['decode_ms'] * 1e3:.0f} tok/s)", flush=True)
    del model
    torch.cuda.empty_cache()
    _compare(cfg, w, prompts, got, 256, first_logits=first)

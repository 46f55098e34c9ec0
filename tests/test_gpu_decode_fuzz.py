"""Seeded random decode cases: every draw picks the GQA shape, batch, lengths (inactive rows,
single keys, page multiples and long contexts), layer geometry, table stride, query and
output dtypes, grid order and split shape from one generator, so combinations that no
targeted test names are still checked.

Plain cases run crucible_attention_decode_paged against the f64 oracle; fused cases run
crucible_attention_decode_paged_append against the reference's three calls (append K,
append V, decode) on copies of the same pools, bit for bit, and then against the oracle on
the appended pools. Every oracle comparison is under the reference's element gate
(gpu_attention_validation.rs:20-22); inactive rows must keep their sentinel.
"""
import numpy as np
import pytest
import torch

import test_gpu_decode as D
from gates import element_gate

pytestmark = pytest.mark.gpu

SEED = 20261202
N_CASES = 48
SHAPES = [(1, 4), (1, 8), (2, 4), (2, 8), (4, 4), (4, 8)]  # (pages per wave, waves)


def _draw(i):
    rng = np.random.default_rng([SEED, i])
    n_kv = int(rng.choice([1, 2, 3, 4, 6, 8, 12]))
    n_rep = int(rng.choice([1, 2, 3, 4, 6, 8, 16]))
    while n_kv * n_rep > 48:  # keeps the oracle's share of the run short
        n_rep //= 2
    batch = int(rng.integers(1, 25))
    max_len = int(rng.choice([16, 100, 700, 2100]))
    lens = rng.integers(1, max_len + 1, size=batch)
    for b in range(batch):
        u = rng.random()
        if u < 0.1:
            lens[b] = 1
        elif u < 0.2:
            lens[b] = 16 * int(rng.integers(1, max(2, max_len // 16 + 1)))
    fused = bool(rng.random() < 0.5)
    if not fused:
        lens[rng.random(batch) < 0.1] = 0  # inactive rows
    n_layer = int(rng.integers(1, 4))
    return {
        "n_kv": n_kv, "n_head": n_kv * n_rep, "lens": [int(n) for n in lens],
        "n_layer": n_layer, "layer": int(rng.integers(0, n_layer)),
        "extra_pages": int(rng.integers(0, 3)),
        "q_f32": bool(rng.random() < 0.3), "out_f16": bool(rng.random() < 0.25),
        "order": [None, "split", "request", "compact"][int(rng.integers(0, 4))],
        "shape": SHAPES[int(rng.integers(0, len(SHAPES)))] if rng.random() < 0.3 else None,
        "fused": fused,
        "positions_seed": int(rng.integers(0, 2**31)),
        "kv_f16": bool(rng.random() < 0.5),
    }


@pytest.mark.parametrize("i", range(N_CASES))
def test_decode_fuzz_case(gpu, dev, tune, i):
    c = _draw(i)
    tune(decode_order=c["order"], decode_pages=c["shape"][0] if c["shape"] else None,
         decode_waves=c["shape"][1] if c["shape"] else None)
    lens, n_head, n_kv = c["lens"], c["n_head"], c["n_kv"]
    what = (f"case {i}: {n_head}/{n_kv} b{len(lens)} max {max(lens)} order {c['order']} "
            f"shape {c['shape']} {'fused' if c['fused'] else 'plain'}")
    print(what, flush=True)
    stride = max(1, -(-max(max(lens), 1) // 16)) + c["extra_pages"]
    if c["fused"]:
        prng = np.random.default_rng(c["positions_seed"])
        positions = [int(prng.integers(0, n)) if prng.random() < 0.3 else n - 1 for n in lens]
        k2, v2, k1, v1, o2, o1, q, tables = D._fused_vs_separate(
            gpu, dev, lens, positions, n_head, n_kv,
            torch.float16 if c["kv_f16"] else torch.float32, n_layer=c["n_layer"],
            layer=c["layer"], seed=SEED + i, stride=stride)
        assert np.array_equal(k2, k1) and np.array_equal(v2, v1), f"{what}: pool bytes differ"
        assert np.array_equal(o2.view(np.uint32), o1.view(np.uint32)), f"{what}: outputs differ"
        want = D._oracle(q.astype(np.float32), k1, v1, tables, lens, n_head, n_kv, c["n_layer"],
                         c["layer"])
        err = element_gate(o2, want, what)
    else:
        q, kp, vp, tables, stride = D._case(SEED + i, lens, n_head, n_kv, n_layer=c["n_layer"],
                                            stride=stride, q_f16=not c["q_f32"])
        got = D._run_decode(gpu, dev, q, kp, vp, tables, lens, n_head, n_kv, c["n_layer"],
                            c["layer"], stride * 16,
                            q_dtype=torch.float32 if c["q_f32"] else torch.float16,
                            out_dtype=torch.float16 if c["out_f16"] else torch.float32)
        active = [b for b, n in enumerate(lens) if n > 0]
        for b, n in enumerate(lens):
            if n <= 0:
                assert np.all(got[b] == np.float32(D.SENTINEL) if not c["out_f16"]
                              else got[b] == np.float16(D.SENTINEL)), f"{what}: row {b} written"
        err = 0.0
        if active:
            want = D._oracle(q, kp, vp, tables, lens, n_head, n_kv, c["n_layer"], c["layer"])
            err = element_gate(got[active], want[active], what, out_f16=c["out_f16"])
    print(f"  max-abs {err:.3e}", flush=True)


def test_draws_cover_the_space():
    """The seeded draws reach every dimension's edges (checked on the host, no GPU work)."""
    cs = [_draw(i) for i in range(N_CASES)]
    assert {c["n_head"] // c["n_kv"] for c in cs} >= {1, 2, 3, 4}
    assert any(1 in c["lens"] for c in cs) and any(0 in c["lens"] for c in cs)
    assert any(max(c["lens"]) > 1024 for c in cs)
    assert {c["order"] for c in cs} == {None, "split", "request", "compact"}
    assert any(c["fused"] for c in cs) and any(not c["fused"] for c in cs)
    assert any(c["q_f32"] for c in cs) and any(c["out_f16"] for c in cs)
    assert any(c["shape"] for c in cs)

"""Hybrid tiled prefill (attention_prefill_tiled with hybrid = 1; gpu.rs:1691-1697,
kernels.cu:2012-2016): keys at or past a segment's absolute_start come from the chunk's own
K/V rows (current_k / current_v, f32, packed like the queries) instead of the pools.

Contracts checked on the reference corpus cases (gpu_attention_validation.rs:431-509):
  * with the chunk's pool slots poisoned (NaN), hybrid gives the bits that the pool path
    gives over the clean pool, when current K/V hold the same fp16 values;
  * with unrounded f32 current K/V, hybrid equals appending those rows through the
    library's packed append (f32 -> fp16, RNE) and running the pool path: bit for bit.
"""
import numpy as np
import pytest
import torch

import attn_cases as A
from gates import element_gate
from test_gpu_prefill import Device, _dev

pytestmark = pytest.mark.gpu

NAN16 = np.uint16(0x7E00)
HYBRID_CASES = [c for c in A.cases()
                if c.name in ("single-1024", "offset-255", "4x256", "ragged-profile-1",
                              "boundary-128", "16x16")]


def _chunk_slots(fx):
    """(row, segment, position, physical page, slot) of every query row's own key."""
    out = []
    for r, (packed, n, start, table) in enumerate(fx.segments):
        for j in range(n):
            pos = start + j
            out.append((packed + j, table, pos, fx.tables[table, pos // 16], pos % 16))
    return out


def _k_index(phys, slot, c):
    return ((phys * A.LAYERS + A.LAYER) * 16 + slot) * A.KD + c


def _v_index(phys, slot, c):
    return ((phys * A.LAYERS + A.LAYER) * 16) * A.KD + c * 16 + slot


def _run(gpu, d, hybrid, cur_k=None, cur_v=None):
    fx = d.fx
    gpu.attention_prefill_tiled(d.q, d.k, d.v, cur_k, cur_v, d.out, d.tables, d.segments,
                                len(fx.case.slices), fx.max_chunk, A.STRIDE, A.HEADS, A.KV_HEADS,
                                A.HD, A.LAYERS, A.LAYER, A.KD, hybrid, 1024)


@pytest.mark.parametrize("case", HYBRID_CASES, ids=lambda c: c.name)
def test_hybrid_reads_the_chunk_from_current_kv(gpu, dev, tune, case):
    tune(prefill_direct=1)  # the pool path in the same kernel the hybrid path takes
    fx = A.fixture(case)
    clean = Device(fx, dev)
    _run(gpu, clean, False)
    want = clean.result().copy()
    # the default precision (P as fp16 hi + lo): the reference's element gate, unwidened
    element_gate(want, A.oracle_out(fx), f"{case.name} pool path")
    # current K/V: the chunk's pool values widened to f32; then poison those pool slots
    cur_k = np.zeros((fx.rows, A.KD), np.float32)
    cur_v = np.zeros((fx.rows, A.KD), np.float32)
    kp, vp = fx.k_pool.copy(), fx.v_pool.copy()
    for row, _, _, phys, slot in _chunk_slots(fx):
        for c in range(A.KD):
            cur_k[row, c] = np.uint16(kp[_k_index(phys, slot, c)]).view(np.float16)
            cur_v[row, c] = np.uint16(vp[_v_index(phys, slot, c)]).view(np.float16)
            kp[_k_index(phys, slot, c)] = NAN16
            vp[_v_index(phys, slot, c)] = NAN16
    d = Device(fx, dev)
    d.k, d.v = _dev(kp, dev), _dev(vp, dev)
    _run(gpu, d, True, _dev(cur_k, dev), _dev(cur_v, dev))
    got = d.result()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), case.name


@pytest.mark.parametrize("case", HYBRID_CASES, ids=lambda c: c.name)
def test_hybrid_rounds_current_kv_like_the_append(gpu, dev, tune, case):
    tune(prefill_direct=1)
    fx = A.fixture(case)
    rng = np.random.default_rng(3)
    cur_k = rng.standard_normal((fx.rows, A.KD)).astype(np.float32) * np.float32(1.7)
    cur_v = rng.standard_normal((fx.rows, A.KD)).astype(np.float32)
    slots = _chunk_slots(fx)
    # pool path: the library's packed append writes the chunk rows, then attention
    d = Device(fx, dev)
    owners = _dev(np.array([s[1] for s in slots], np.int32), dev)
    positions = _dev(np.array([s[2] for s in slots], np.int32), dev)
    rows = np.array([s[0] for s in slots])
    d_ck, d_cv = _dev(cur_k[rows], dev), _dev(cur_v[rows], dev)
    gpu.cache_store_packed_paged(d_ck, d.k, d.tables, owners, positions, len(slots), A.KD,
                                 A.STRIDE, A.LAYERS, A.LAYER, kind="k")
    gpu.cache_store_packed_paged(d_cv, d.v, d.tables, owners, positions, len(slots), A.KD,
                                 A.STRIDE, A.LAYERS, A.LAYER, kind="v")
    _run(gpu, d, False)
    want = d.result().copy()
    # hybrid over a pool whose chunk slots hold NaN
    kp, vp = fx.k_pool.copy(), fx.v_pool.copy()
    for _, _, _, phys, slot in slots:
        for c in range(A.KD):
            kp[_k_index(phys, slot, c)] = NAN16
            vp[_v_index(phys, slot, c)] = NAN16
    h = Device(fx, dev)
    h.k, h.v = _dev(kp, dev), _dev(vp, dev)
    _run(gpu, h, True, _dev(cur_k, dev), _dev(cur_v, dev))
    got = h.result()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), case.name


@pytest.mark.parametrize("case", HYBRID_CASES, ids=lambda c: c.name)
def test_hybrid_ignores_table_entries_of_chunk_pages(gpu, dev, tune, case):
    """The reference never reads the table or the pool for keys at or past absolute_start
    (kernels.cu:2012-2016), so a table whose entries for pages wholly inside the chunk are
    not yet the chunk's pages must give the same bits. Here those entries all name page 0
    (a valid page, so every address stays inside the pool) and the output is unchanged."""
    for direct in (1, None):  # the register-direct kernel, and the launcher's own choice
        tune(prefill_direct=direct)
        fx = A.fixture(case)
        rng = np.random.default_rng(5)
        cur_k = rng.standard_normal((fx.rows, A.KD)).astype(np.float32)
        cur_v = rng.standard_normal((fx.rows, A.KD)).astype(np.float32)
        d = Device(fx, dev)
        _run(gpu, d, True, _dev(cur_k, dev), _dev(cur_v, dev))
        want = d.result().copy()
        tables = fx.tables.copy()
        changed = 0
        for packed, n, start, table in fx.segments:
            for page in range(-(-int(start) // 16), -(-int(start + n) // 16)):
                tables[table, page] = 0
                changed += 1
        assert changed > 0
        d2 = Device(fx, dev)
        d2.tables = _dev(tables, dev)
        _run(gpu, d2, True, _dev(cur_k, dev), _dev(cur_v, dev))
        got = d2.result()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), case.name

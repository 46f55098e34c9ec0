"""Pins the oracle's page geometry and KV-append scatters.

Checks: the reference's geometry KATs (engine/src/paged.rs:267-274), the closed form of
kernels.cu:1630-1638, brute-force element placement, append -> gather round trips for all
four reference scatters, and the V block transpose against the reference element order.
"""
import numpy as np
import pytest

import oracle

N_LAYER, KV_DIM = 12, 192


def test_paged_offset_closed_form():
    rng = np.random.default_rng(1)
    for _ in range(1000):
        page, slot, layer = int(rng.integers(0, 8192)), int(rng.integers(0, 16)), int(rng.integers(0, 12))
        kv = int(rng.choice([64, 192, 256, 768]))
        want = page * 12 * 16 * kv + layer * 16 * kv + slot * kv
        assert oracle.paged_offset(page, slot, 12, layer, kv) == want


def test_paged_offset_is_64_bit():
    # page * n_layer * 16 * kv_dim overflows int32 for large pools (H5): 8191*12*16*768
    assert oracle.paged_offset(8191, 15, 12, 11, 768) == ((8191 * 12 + 11) * 16 + 15) * 768
    assert oracle.paged_offset(300000, 0, 24, 0, 1024) > 2 ** 31


def test_page_geometry_matches_layout():
    # paged.rs:267-274: one page holds n_layer * 16 * kv_dim elements; 64 pages == 1024 tokens
    assert oracle.paged_offset(1, 0, N_LAYER, 0, KV_DIM) == N_LAYER * 16 * KV_DIM
    assert oracle.paged_offset(64, 0, N_LAYER, 0, KV_DIM) == N_LAYER * 1024 * KV_DIM


def test_v_index_is_block_transpose_of_k_index():
    for page, slot, c, layer in [(0, 0, 0, 0), (3, 5, 100, 7), (17, 15, 191, 11)]:
        k = oracle.pool_index(oracle.POOL_K, page, slot, c, N_LAYER, layer, KV_DIM)
        v = oracle.pool_index(oracle.POOL_V, page, slot, c, N_LAYER, layer, KV_DIM)
        block = oracle.paged_offset(page, 0, N_LAYER, layer, KV_DIM)
        assert k == block + slot * KV_DIM + c
        assert v == block + c * 16 + slot


def _pool(n_pages, n_layer=N_LAYER, kv=KV_DIM):
    return np.full(n_pages * n_layer * 16 * kv, 0x7E00, np.uint16)  # NaN everywhere


@pytest.mark.parametrize("kind", [oracle.POOL_K, oracle.POOL_V])
def test_rows_append_places_every_element(kind):
    rng = np.random.default_rng(2)
    n_pages, stride, rows = 20, 4, 5
    tables = rng.permutation(n_pages)[: rows * stride].reshape(rows, stride).astype(np.int32)
    positions = rng.integers(0, stride * 16, rows).astype(np.int32)
    src = rng.standard_normal((rows, KV_DIM)).astype(np.float32)
    pool = _pool(n_pages)
    oracle.cache_store(oracle.STORE_ROWS, kind, pool, src, tables=tables, positions=positions,
                       rows=rows, kv_dim=KV_DIM, table_stride=stride, n_layer=N_LAYER, layer=3)
    h = src.astype(np.float16).view(np.uint16)
    touched = 0
    for r in range(rows):
        page = tables[r, positions[r] >> 4]
        for c in range(KV_DIM):
            idx = oracle.pool_index(kind, int(page), int(positions[r] & 15), c, N_LAYER, 3, KV_DIM)
            assert pool[idx] == h[r, c]
            touched += 1
    assert np.count_nonzero(pool != 0x7E00) == touched


def test_all_store_modes_round_trip_through_gather():
    rng = np.random.default_rng(3)
    n_pages, stride, n_layer, layer, kv = 30, 6, 3, 1, 128
    lens = [37, 90]
    perm = rng.permutation(n_pages).astype(np.int32)
    tables = np.zeros((2, stride), np.int32)
    tables[0, :3] = perm[:3]
    tables[1, :6] = perm[3:9]
    for kind in (oracle.POOL_K, oracle.POOL_V):
        dense = [rng.standard_normal((L, kv)).astype(np.float32) for L in lens]
        # PACKED: both sequences in one buffer
        pool = _pool(n_pages, n_layer, kv)
        owners = np.concatenate([np.full(L, i, np.int32) for i, L in enumerate(lens)])
        pos = np.concatenate([np.arange(L, dtype=np.int32) for L in lens])
        oracle.cache_store(oracle.STORE_PACKED, kind, pool, np.concatenate(dense), tables=tables,
                           owners=owners, positions=pos, rows=len(pos), kv_dim=kv,
                           table_stride=stride, n_layer=n_layer, layer=layer)
        for i, L in enumerate(lens):
            got = oracle.gather(kind, pool, tables[i], L, kv, n_layer, layer)
            assert np.array_equal(got, dense[i].astype(np.float16).astype(np.float32))
        # PARAMS: sequence 1 in two chunks, second chunk at params[5] = 40
        pool = _pool(n_pages, n_layer, kv)
        for start, stop in ((0, 40), (40, 90)):
            params = np.array([0, 0, 0, 0, 0, start], np.int32)
            oracle.cache_store(oracle.STORE_PARAMS, kind, pool, dense[1][start:stop],
                               tables=tables[1], params=params, rows=stop - start, kv_dim=kv,
                               n_layer=n_layer, layer=layer)
        got = oracle.gather(kind, pool, tables[1], 90, kv, n_layer, layer)
        assert np.array_equal(got, dense[1].astype(np.float16).astype(np.float32))
        # ROWS: one token per sequence, per step
        pool = _pool(n_pages, n_layer, kv)
        for t in range(37):
            oracle.cache_store(oracle.STORE_ROWS, kind, pool,
                               np.stack([dense[0][t], dense[1][t]]), tables=tables,
                               positions=np.array([t, t], np.int32), rows=2, kv_dim=kv,
                               table_stride=stride, n_layer=n_layer, layer=layer)
        for i in range(2):
            got = oracle.gather(kind, pool, tables[i], 37, kv, n_layer, layer)
            assert np.array_equal(got, dense[i][:37].astype(np.float16).astype(np.float32))


def test_contiguous_store_equals_paged_with_identity_table():
    rng = np.random.default_rng(4)
    cap, n_layer, layer, kv = 64, 2, 1, 64
    src = rng.standard_normal((50, kv)).astype(np.float32)
    for kind in (oracle.POOL_K, oracle.POOL_V):
        contig = np.zeros(n_layer * cap * kv, np.uint16)
        oracle.cache_store(oracle.STORE_CONTIG, kind, contig, src, rows=50, kv_dim=kv,
                           layer_base=layer * cap * kv, pos_offset=5)
        # a contiguous layer region is a paged pool of cap/16 pages, n_layer = 1
        region = contig[layer * cap * kv:(layer + 1) * cap * kv]
        ident = np.arange(cap // 16, dtype=np.int32)
        got = oracle.gather(kind, region, ident, 55, kv, 1, 0)
        assert np.array_equal(got[5:], src.astype(np.float16).astype(np.float32))


def test_v_blocks_transpose_round_trip_and_reference_order():
    rng = np.random.default_rng(5)
    kv, n_pages, n_layer = 192, 3, 2
    ref = rng.integers(0, 65535, n_pages * n_layer * 16 * kv).astype(np.uint16)
    vt = oracle.v_blocks_from_reference(ref, kv)
    assert np.array_equal(oracle.v_blocks_to_reference(vt, kv), ref)
    blocks = ref.reshape(n_pages * n_layer, 16, kv)
    assert np.array_equal(vt.reshape(n_pages * n_layer, kv, 16), blocks.transpose(0, 2, 1))

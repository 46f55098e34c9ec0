"""Pins the attention oracle itself (no GPU).

Against: torch's scaled_dot_product_attention in float64 (a library routine; the call the
reference's model.py:205-211 makes, including enable_gqa's h // n_rep grouping), a numpy
textbook restatement, closed forms (zero query -> mean of V, one key -> that value,
dominant score -> its value), and the split-K algebra of kernels.cu:692-850.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle


def _sdpa_f64(q, k, v, n_head, n_kv, hd, causal):
    """q [T, n_head*hd], k/v [S, n_kv*hd] -> [T, n_head*hd] via torch SDPA (float64)."""
    T, S = q.shape[0], k.shape[0]
    qt = torch.from_numpy(q.astype(np.float64)).view(1, T, n_head, hd).transpose(1, 2)
    kt = torch.from_numpy(k.astype(np.float64)).view(1, S, n_kv, hd).transpose(1, 2)
    vt = torch.from_numpy(v.astype(np.float64)).view(1, S, n_kv, hd).transpose(1, 2)
    if n_kv != n_head:  # repeat_interleave: kv head j -> query heads [j*n_rep, (j+1)*n_rep)
        kt = kt.repeat_interleave(n_head // n_kv, dim=1)
        vt = vt.repeat_interleave(n_head // n_kv, dim=1)
    mask = None
    if causal:  # query i sits at absolute position S - T + i
        mask = torch.ones(T, S, dtype=torch.bool).tril(diagonal=S - T)
    y = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask)
    return y.transpose(1, 2).reshape(T, n_head * hd).numpy()


@pytest.mark.parametrize("n_head,n_kv", [(12, 3), (12, 12), (16, 4), (12, 1), (12, 6)])
def test_dense_oracle_matches_torch_sdpa(n_head, n_kv):
    rng = np.random.default_rng(n_head * 100 + n_kv)
    hd, T, S = 64, 40, 100
    q = rng.standard_normal((T, n_head * hd)).astype(np.float32)
    k = rng.standard_normal((S, n_kv * hd)).astype(np.float32)
    v = rng.standard_normal((S, n_kv * hd)).astype(np.float32)
    lens = np.arange(S - T + 1, S + 1, dtype=np.int32)          # causal, last T positions
    got = oracle.attention_dense(q, k, v, lens, n_head, n_kv, hd)
    want = _sdpa_f64(q, k, v, n_head, n_kv, hd, causal=True)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)


def test_dense_oracle_matches_numpy_textbook():
    rng = np.random.default_rng(9)
    n_head, n_kv, hd, S = 8, 2, 64, 33
    q = rng.standard_normal((1, n_head * hd)).astype(np.float32)
    k = rng.standard_normal((S, n_kv * hd)).astype(np.float32)
    v = rng.standard_normal((S, n_kv * hd)).astype(np.float32)
    got = oracle.attention_dense(q, k, v, np.array([S], np.int32), n_head, n_kv, hd)[0]
    for h in range(n_head):
        g = h // (n_head // n_kv)
        s = (k[:, g * hd:(g + 1) * hd].astype(np.float64) @ q[0, h * hd:(h + 1) * hd]) / 8.0
        p = np.exp(s - s.max())
        p /= p.sum()
        o = p @ v[:, g * hd:(g + 1) * hd].astype(np.float64)
        np.testing.assert_allclose(got[h * hd:(h + 1) * hd], o, rtol=1e-6, atol=1e-7)


def test_closed_forms():
    rng = np.random.default_rng(10)
    hd, S = 64, 50
    k = rng.standard_normal((S, hd)).astype(np.float32)
    v = rng.standard_normal((S, hd)).astype(np.float32)
    # zero query: uniform weights, output is the mean of the visible values
    out = oracle.attention_dense(np.zeros((1, hd), np.float32), k, v, np.array([S], np.int32), 1, 1, hd)
    np.testing.assert_allclose(out[0], v.astype(np.float64).mean(0), rtol=1e-6, atol=1e-7)
    # one visible key: output is exactly that value
    q = rng.standard_normal((1, hd)).astype(np.float32)
    out = oracle.attention_dense(q, k, v, np.array([1], np.int32), 1, 1, hd)
    assert np.array_equal(out[0], v[0])
    # a dominant score: key 17 aligned with the query and scaled up
    kd = k.copy()
    kd[17] = q[0] * 40.0
    out = oracle.attention_dense(q, kd, v, np.array([S], np.int32), 1, 1, hd)
    np.testing.assert_allclose(out[0], v[17], atol=1e-6)


def test_reference_order_f32_agrees_with_f64():
    """model.rs-order f32 attention vs the f64 definition, within 1e-5."""
    rng = np.random.default_rng(11)
    n_head, n_kv, hd, S = 12, 3, 64, 1024
    q = rng.standard_normal((4, n_head * hd)).astype(np.float32)
    k = rng.standard_normal((S, n_kv * hd)).astype(np.float32)
    v = rng.standard_normal((S, n_kv * hd)).astype(np.float32)
    lens = np.array([1, 17, 512, 1024], np.int32)
    a = oracle.attention_dense(q, k, v, lens, n_head, n_kv, hd, precise=True)
    b = oracle.attention_dense(q, k, v, lens, n_head, n_kv, hd, precise=False)
    assert np.abs(a - b).max() <= 1e-5


def test_split_combine_equals_unsplit_and_empty_chunks_are_neutral():
    rng = np.random.default_rng(12)
    hd, cap = 64, 1024
    q = rng.standard_normal(hd).astype(np.float32)
    k = rng.standard_normal((cap, hd)).astype(np.float32) * 2
    v = rng.standard_normal((cap, hd)).astype(np.float32)
    for length in (1, 127, 128, 129, 700, 1024):
        n_chunks = cap // 128
        pm, pl, po = oracle.split_partials(q, k, v, length, hd, 128, n_chunks)
        used = -(-length // 128)
        assert np.all(np.isneginf(pm[used:])) and np.all(pl[used:] == 0) and np.all(po[used:] == 0)
        got = oracle.split_combine(pm, pl, po)
        want = oracle.attention_dense(q[None], k, v, np.array([length], np.int32), 1, 1, hd)[0]
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)


def test_paged_rows_equals_dense_on_gathered_history():
    rng = np.random.default_rng(13)
    n_head, n_kv, hd, n_layer, layer = 12, 3, 64, 3, 1
    kv = n_kv * hd
    n_pages, stride = 40, 8
    k_pool = oracle.f32_to_f16_bits(rng.standard_normal(n_pages * n_layer * 16 * kv))
    v_pool = oracle.f32_to_f16_bits(rng.standard_normal(n_pages * n_layer * 16 * kv))
    tables = rng.permutation(n_pages)[:2 * stride].reshape(2, stride).astype(np.int32)
    lens = np.array([100, 7], np.int32)
    q = rng.standard_normal((2, n_head * hd)).astype(np.float32)
    got = oracle.attention_paged_rows(q, k_pool, v_pool, tables, lens, n_head=n_head,
                                      n_kv_head=n_kv, head_dim=hd, table_stride=stride,
                                      n_layer=n_layer, layer=layer)
    for b in range(2):
        kd = oracle.gather(oracle.POOL_K, k_pool, tables[b], lens[b], kv, n_layer, layer)
        vd = oracle.gather(oracle.POOL_V, v_pool, tables[b], lens[b], kv, n_layer, layer)
        want = _sdpa_f64(q[b:b + 1], kd, vd, n_head, n_kv, hd, causal=False)
        np.testing.assert_allclose(got[b], want[0], rtol=1e-6, atol=1e-6)


def test_future_positions_never_read():
    """Poisoning everything at or past len leaves the output bit-identical (kernels read < len)."""
    rng = np.random.default_rng(14)
    n_head, n_kv, hd, n_layer, kv = 4, 1, 64, 1, 64
    k_pool = oracle.f32_to_f16_bits(rng.standard_normal(8 * 16 * kv))
    v_pool = oracle.f32_to_f16_bits(rng.standard_normal(8 * 16 * kv))
    table = np.arange(8, dtype=np.int32)[None]
    q = rng.standard_normal((1, n_head * hd)).astype(np.float32)
    length = 37
    a = oracle.attention_paged_rows(q, k_pool, v_pool, table, [length], n_head=n_head,
                                    n_kv_head=n_kv, head_dim=hd, table_stride=8, n_layer=1, layer=0)
    kp, vp = k_pool.copy(), v_pool.copy()
    poison = int(oracle.f32_to_f16_bits(np.array([123.75], np.float32))[0])
    for p in range(length, 8 * 16):
        for c in range(kv):
            kp[oracle.pool_index(0, p >> 4, p & 15, c, 1, 0, kv)] = poison
            vp[oracle.pool_index(1, p >> 4, p & 15, c, 1, 0, kv)] = 0x7E00  # NaN
    b = oracle.attention_paged_rows(q, kp, vp, table, [length], n_head=n_head, n_kv_head=n_kv,
                                    head_dim=hd, table_stride=8, n_layer=1, layer=0)
    assert np.array_equal(a, b)

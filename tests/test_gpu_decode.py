"""Paged decode parity against the f64 oracle, plus the reference's structural contracts:
inactive requests untouched, future slots never read, paged == contiguous bit for bit, page
remapping and batch order invariant. Every oracle comparison asserts the reference's element
gate (|d| <= 2e-5 + 2e-5 |ref|, gpu_attention_validation.rs:20-22) and the north-star max-abs
2e-3 (tests/gates.py)."""
import numpy as np
import pytest
import torch

import oracle
from attn_cases import disjoint_tables, random_pools
from gates import element_gate

pytestmark = pytest.mark.gpu

SENTINEL = -12345.25
ORDERS = ["split", "request", "compact"]  # decode_order tuning values


def _dev(a, dev):
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.float16).copy()).to(dev)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _run_decode(gpu, dev, q, k_pool, v_pool, tables, lens, n_head, n_kv, n_layer, layer,
                max_seq, q_dtype=torch.float16, out_dtype=torch.float32):
    batch, stride = tables.shape
    kv = n_kv * 64
    d_q = torch.from_numpy(q).to(dev).to(q_dtype)
    out = torch.full((batch, n_head * 64), SENTINEL, dtype=out_dtype, device=dev)
    gpu.attention_decode_paged(d_q, _dev(k_pool, dev), _dev(v_pool, dev), out, _dev(tables, dev),
                               _dev(np.asarray(lens, np.int32), dev), batch, n_head, n_kv, 64,
                               stride, n_layer, layer, kv, max_seq)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def _case(seed, lens, n_head, n_kv, n_layer=3, stride=None, q_f16=True):
    rng = np.random.default_rng(seed)
    stride = stride or max(1, -(-max(max(lens), 1) // 16))
    n_pages = sum(-(-max(n, 1) // 16) for n in lens) + 4
    k_pool, v_pool = random_pools(rng, n_pages, n_layer, n_kv * 64)
    tables = disjoint_tables(rng, n_pages, [max(n, 1) for n in lens], stride)
    q = rng.standard_normal((len(lens), n_head * 64)).astype(np.float32)
    if q_f16:
        q = q.astype(np.float16).astype(np.float32)
    return q, k_pool, v_pool, tables, stride


def _oracle(q, k_pool, v_pool, tables, lens, n_head, n_kv, n_layer, layer):
    lens = np.asarray(lens, np.int32)
    return oracle.attention_paged_rows(q, k_pool, v_pool, tables, lens, n_head=n_head,
                                       n_kv_head=n_kv, head_dim=64,
                                       table_stride=tables.shape[1], n_layer=n_layer, layer=layer)


EDGE_LENS = [1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 511, 512, 1023, 1024, 2048]


@pytest.mark.parametrize("n_head,n_kv", [(12, 3), (12, 12), (16, 4), (12, 6), (12, 1), (16, 16)])
def test_decode_matches_oracle_across_page_boundaries(gpu, dev, n_head, n_kv):
    lens = EDGE_LENS
    q, kp, vp, tables, stride = _case(n_head * 31 + n_kv, lens, n_head, n_kv)
    got = _run_decode(gpu, dev, q, kp, vp, tables, lens, n_head, n_kv, 3, 1, stride * 16)
    want = _oracle(q, kp, vp, tables, lens, n_head, n_kv, 3, 1)
    err = element_gate(got, want, f"decode {n_head}/{n_kv}")
    print(f"decode {n_head}/{n_kv}: max-abs {err:.3e}")


@pytest.mark.parametrize("q_dtype,out_dtype", [(torch.float32, torch.float32),
                                               (torch.float16, torch.float16),
                                               (torch.float32, torch.float16)])
def test_decode_dtypes(gpu, dev, q_dtype, out_dtype):
    lens = [7, 300, 1000]
    q, kp, vp, tables, stride = _case(3, lens, 12, 3, q_f16=False)
    got = _run_decode(gpu, dev, q, kp, vp, tables, lens, 12, 3, 3, 1, stride * 16,
                      q_dtype=q_dtype, out_dtype=out_dtype)
    qq = q if q_dtype == torch.float32 else q.astype(np.float16).astype(np.float32)
    want = _oracle(qq, kp, vp, tables, lens, 12, 3, 3, 1)
    # an fp16 output adds its own rounding; an f32 query is carried as hi + lo fp16 halves
    element_gate(got, want, f"decode {q_dtype} -> {out_dtype}",
                 out_f16=out_dtype == torch.float16)


def test_inactive_requests_are_untouched(gpu, dev):
    lens = [0, 50, 0, -3, 200]
    q, kp, vp, tables, stride = _case(4, lens, 12, 3)
    got = _run_decode(gpu, dev, q, kp, vp, tables, lens, 12, 3, 3, 1, stride * 16)
    for b in (0, 2, 3):
        assert np.all(got[b] == SENTINEL)
    want = _oracle(q, kp, vp, tables, lens, 12, 3, 3, 1)
    element_gate(got[[1, 4]], want[[1, 4]], "active requests")


def test_future_slots_are_never_read(gpu, dev):
    """NaN in every slot at or past seq_len (same page and later pages) changes nothing."""
    lens = [37, 16, 129]
    n_layer, layer, kv = 3, 1, 192
    q, kp, vp, tables, stride = _case(5, lens, 12, 3, stride=16)
    clean = _run_decode(gpu, dev, q, kp, vp, tables, lens, 12, 3, n_layer, layer, stride * 16)
    kp2, vp2 = kp.copy(), vp.copy()
    for b, n in enumerate(lens):
        for pos in range(n, -(-n // 16) * 16):
            page = tables[b, pos >> 4]
            for c in range(kv):
                kp2[oracle.pool_index(0, page, pos & 15, c, n_layer, layer, kv)] = 0x7E00
                vp2[oracle.pool_index(1, page, pos & 15, c, n_layer, layer, kv)] = 0x7E00
    # pages after the last one in the table: point them at a NaN-filled page
    poisoned = _run_decode(gpu, dev, q, kp2, vp2, tables, lens, 12, 3, n_layer, layer, stride * 16)
    assert np.array_equal(clean.view(np.uint32), poisoned.view(np.uint32))


def test_page_remap_and_batch_order_invariance(gpu, dev):
    lens = [100, 1, 700, 33]
    n_layer, layer, kv = 2, 0, 192
    q, kp, vp, tables, stride = _case(6, lens, 12, 3, n_layer=n_layer)
    base = _run_decode(gpu, dev, q, kp, vp, tables, lens, 12, 3, n_layer, layer, stride * 16)
    # move every used page to a new physical id (same contents)
    rng = np.random.default_rng(60)
    n_pages = kp.size // (n_layer * 16 * kv)
    perm = rng.permutation(n_pages)
    blk = n_layer * 16 * kv
    kp2 = np.empty_like(kp)
    vp2 = np.empty_like(vp)
    for old in range(n_pages):
        kp2[perm[old] * blk:(perm[old] + 1) * blk] = kp[old * blk:(old + 1) * blk]
        vp2[perm[old] * blk:(perm[old] + 1) * blk] = vp[old * blk:(old + 1) * blk]
    tables2 = perm[tables].astype(np.int32)
    remapped = _run_decode(gpu, dev, q, kp2, vp2, tables2, lens, 12, 3, n_layer, layer, stride * 16)
    assert np.array_equal(base.view(np.uint32), remapped.view(np.uint32))
    order = [2, 0, 3, 1]
    shuffled = _run_decode(gpu, dev, q[order], kp, vp, tables[order], [lens[i] for i in order],
                           12, 3, n_layer, layer, stride * 16)
    assert np.array_equal(base[order].view(np.uint32), shuffled.view(np.uint32))


def test_paged_equals_contiguous_bit_for_bit(gpu, dev):
    """The reference's gpu-paged contract (main.rs:1253-1257) for decode."""
    rng = np.random.default_rng(7)
    n_head, n_kv, hd, kv, cap, n_layer, layer = 12, 3, 64, 192, 1024, 3, 2
    for length in [1, 7, 15, 16, 17, 31, 32, 33, 64, 127, 128, 129, 256, 511, 512, 1023]:
        # contiguous cache [layer][cap][kv] (V: [layer][cap/16][kv][16]) ...
        k_c, v_c = random_pools(rng, cap // 16, n_layer, kv)  # same element count
        # ... equals a pool whose page p (one layer) is block p of the layer region
        q = rng.standard_normal((1, n_head * hd)).astype(np.float16)
        params = np.array([0, 0, length - 1, length, 0, 0], np.int32)
        out_c = torch.zeros((1, n_head * hd), dtype=torch.float32, device=dev)
        gpu.attention_decode(_dev(q, dev), _dev(k_c, dev), _dev(v_c, dev), out_c, n_head, n_kv,
                             hd, _dev(params, dev), cap, kv, layer * cap * kv)
        region = slice(layer * cap * kv, (layer + 1) * cap * kv)
        k_p, v_p = k_c[region].copy(), v_c[region].copy()
        table = rng.permutation(cap // 16).astype(np.int32)
        k_perm, v_perm = np.empty_like(k_p), np.empty_like(v_p)
        blk = 16 * kv
        for logical in range(cap // 16):
            phys = table[logical]
            k_perm[phys * blk:(phys + 1) * blk] = k_p[logical * blk:(logical + 1) * blk]
            v_perm[phys * blk:(phys + 1) * blk] = v_p[logical * blk:(logical + 1) * blk]
        out_p = torch.zeros_like(out_c)
        gpu.attention_decode_paged(_dev(q, dev), _dev(k_perm, dev), _dev(v_perm, dev), out_p,
                                   _dev(table[None], dev), _dev(np.array([length], np.int32), dev),
                                   1, n_head, n_kv, hd, cap // 16, 1, 0, kv, cap)
        torch.cuda.synchronize()
        assert torch.equal(out_c, out_p), length


def test_split_form_matches_oracle(gpu, dev):
    """attention_split (caller-owned partials, 128-token chunks) on a contiguous cache."""
    rng = np.random.default_rng(8)
    n_head, n_kv, hd, kv, cap = 12, 3, 64, 192, 1024
    k_c, v_c = random_pools(rng, cap // 16, 1, kv)
    for length in [1, 128, 129, 777, 1024]:
        q = rng.standard_normal((1, n_head * hd)).astype(np.float32)
        params = np.array([0, 0, length - 1, length, 0, 0], np.int32)
        n_chunks = cap // 128
        po = torch.zeros(n_head * n_chunks * hd, device=dev)
        pm = torch.zeros(n_head * n_chunks, device=dev)
        pl = torch.zeros(n_head * n_chunks, device=dev)
        out = torch.zeros((1, n_head * hd), device=dev)
        gpu.attention_split(_dev(q, dev), _dev(k_c, dev), _dev(v_c, dev), po, pm, pl, out, n_head,
                            n_kv, hd, _dev(params, dev), cap, kv, 0)
        torch.cuda.synchronize()
        want = _oracle(q, k_c, v_c, np.arange(cap // 16, dtype=np.int32)[None], [length], n_head,
                       n_kv, 1, 0)
        element_gate(out.cpu().numpy(), want, f"attention_split len {length}")


def test_config2_decode_b1_ctx1024(gpu, dev):
    from crucible_amd.workloads import config2_decode_b1
    for n_kv in (3, 12):
        cfg = config2_decode_b1(n_kv_head=n_kv)
        rng = np.random.default_rng(cfg.seed)
        kp, vp = random_pools(rng, cfg.n_pages, cfg.n_layer, cfg.kv_dim)
        q = rng.standard_normal((1, 12 * 64)).astype(np.float16).astype(np.float32)
        got = _run_decode(gpu, dev, q, kp, vp, cfg.tables, cfg.lens, 12, n_kv, cfg.n_layer, 0,
                          cfg.max_seq)
        want = _oracle(q, kp, vp, cfg.tables, cfg.lens, 12, n_kv, cfg.n_layer, 0)
        element_gate(got, want, f"config 2, {n_kv} kv heads")


def test_config3_decode_b16_all_layers(gpu, dev):
    """BASELINE config 3 at full size (8192-page pool, 12 layers, ctx 65..2048), GQA-3."""
    from crucible_amd.workloads import config3_decode_b16, make_pools
    cfg = config3_decode_b16()
    rng = np.random.default_rng(cfg.seed)
    tables = disjoint_tables(rng, cfg.n_pages, cfg.lens, cfg.table_stride)
    kp, vp = make_pools(cfg.n_pages, cfg.n_layer, cfg.kv_dim, cfg.seed, dev)
    # compact copy of the used pages for the oracle
    used = np.unique(np.concatenate([tables[b, :-(-int(n) // 16)] for b, n in enumerate(cfg.lens)]))
    remap = np.zeros(cfg.n_pages, np.int32)
    remap[used] = np.arange(used.size, dtype=np.int32)
    blk = cfg.n_layer * 16 * cfg.kv_dim
    idx = torch.from_numpy(used).long().to(dev)
    kc = kp.view(cfg.n_pages, blk)[idx].cpu().numpy().view(np.uint16).reshape(-1)
    vc = vp.view(cfg.n_pages, blk)[idx].cpu().numpy().view(np.uint16).reshape(-1)
    ctables = remap[tables]
    q_all = torch.randn(cfg.n_layer, 16, 12 * 64, device=dev).to(torch.float16)
    out = torch.zeros(16, 12 * 64, device=dev)
    d_tab, d_len = _dev(tables, dev), _dev(cfg.lens, dev)
    worst = 0.0
    for layer in range(cfg.n_layer):
        gpu.attention_decode_paged(q_all[layer], kp, vp, out, d_tab, d_len, 16, 12, 3, 64,
                                   cfg.table_stride, cfg.n_layer, layer, cfg.kv_dim, cfg.max_seq)
        torch.cuda.synchronize()
        want = _oracle(q_all[layer].float().cpu().numpy(), kc, vc, ctables, cfg.lens, 12, 3,
                       cfg.n_layer, layer)
        worst = max(worst, element_gate(out.cpu().numpy(), want, f"config 3 layer {layer}"))
    print(f"config3 all layers: max-abs {worst:.3e}")


# ---------------------------------------------------------------- fused append + decode

def _fused_vs_separate(gpu, dev, lens, positions, n_head, n_kv, kv_dtype=torch.float32,
                       n_layer=3, layer=1, seed=0, stride=None, shapes=None):
    """Run the fused entry and the reference's three calls on copies of the same pools;
    return (fused pools, separate pools, fused out, separate out) as host arrays."""
    rng = np.random.default_rng(seed)
    batch = len(lens)
    kv = n_kv * 64
    stride = stride or max(1, -(-max(max(lens), max(positions) + 1, 1) // 16))
    need = [max(-(-max(n, 1) // 16), (p >> 4) + 1) for n, p in zip(lens, positions)]
    n_pages = sum(need) + 3
    kp, vp = random_pools(rng, n_pages, n_layer, kv)
    tables = disjoint_tables(rng, n_pages, [16 * k for k in need], stride)
    q = rng.standard_normal((batch, n_head * 64)).astype(np.float16)
    k_new = (rng.standard_normal((batch, kv)) * 2).astype(np.float32)
    v_new = (rng.standard_normal((batch, kv)) * 2).astype(np.float32)
    d_q = _dev(q, dev)
    d_tab = _dev(tables, dev)
    d_pos = _dev(np.asarray(positions, np.int32), dev)
    d_len = _dev(np.asarray(lens, np.int32), dev)
    d_kn = torch.from_numpy(k_new).to(dev).to(kv_dtype)
    d_vn = torch.from_numpy(v_new).to(dev).to(kv_dtype)
    max_seq = stride * 16
    # separate: append K, append V, decode
    k1, v1 = _dev(kp, dev), _dev(vp, dev)
    out1 = torch.full((batch, n_head * 64), SENTINEL, device=dev)
    gpu.cache_store_rows_paged(d_kn, k1, d_tab, d_pos, batch, kv, stride, n_layer, layer, kind="k")
    gpu.cache_store_rows_paged(d_vn, v1, d_tab, d_pos, batch, kv, stride, n_layer, layer, kind="v")
    gpu.attention_decode_paged(d_q, k1, v1, out1, d_tab, d_len, batch, n_head, n_kv, 64, stride,
                               n_layer, layer, kv, max_seq)
    # fused
    k2, v2 = _dev(kp, dev), _dev(vp, dev)
    out2 = torch.full((batch, n_head * 64), SENTINEL, device=dev)
    gpu.attention_decode_paged_append(d_q, d_kn, d_vn, k2, v2, out2, d_tab, d_pos, d_len, batch,
                                      n_head, n_kv, 64, stride, n_layer, layer, kv, max_seq)
    torch.cuda.synchronize()
    return (k2.cpu().numpy().view(np.uint16), v2.cpu().numpy().view(np.uint16),
            k1.cpu().numpy().view(np.uint16), v1.cpu().numpy().view(np.uint16),
            out2.cpu().numpy(), out1.cpu().numpy(), q, tables)


@pytest.mark.parametrize("n_head,n_kv", [(12, 3), (12, 12), (16, 4), (12, 1)])
@pytest.mark.parametrize("kv_dtype", [torch.float32, torch.float16])
def test_fused_append_decode_equals_separate_calls(gpu, dev, n_head, n_kv, kv_dtype):
    lens = [1, 15, 16, 17, 32, 33, 255, 256, 257, 700, 1024, 2048]
    positions = [n - 1 for n in lens]
    k2, v2, k1, v1, o2, o1, q, tables = _fused_vs_separate(
        gpu, dev, lens, positions, n_head, n_kv, kv_dtype, seed=n_head + n_kv)
    assert np.array_equal(k2, k1) and np.array_equal(v2, v1), "pool bytes differ"
    assert np.array_equal(o2.view(np.uint32), o1.view(np.uint32)), "outputs differ"
    # and both match the oracle on the appended pools
    want = _oracle(q.astype(np.float32), k1, v1, tables, lens, n_head, n_kv, 3, 1)
    element_gate(o2, want, f"fused {n_head}/{n_kv} {kv_dtype}")


@pytest.mark.parametrize("order", ORDERS)
def test_fused_append_off_the_last_slot_and_inactive_rows(gpu, dev, tune, order):
    """Rows appended inside the attended range, past it (a later page, and a later split:
    a unit of its own in the compact order), and for inactive requests (len 0) give the
    same pools and outputs as the separate calls."""
    tune(decode_order=order)
    lens = [40, 40, 0, 300, 17, 129, 0]
    positions = [20, 100, 5, 299, 16, 128, 700]
    for rep in range(3):  # repeated launches reuse the workspace counters
        k2, v2, k1, v1, o2, o1, _, _ = _fused_vs_separate(gpu, dev, lens, positions, 12, 3,
                                                          seed=70 + rep)
        assert np.array_equal(k2, k1) and np.array_equal(v2, v1)
        active = [b for b, n in enumerate(lens) if n > 0]
        assert np.array_equal(o2[active].view(np.uint32), o1[active].view(np.uint32))
        assert np.all(o2[2] == SENTINEL)


@pytest.mark.parametrize("order", ORDERS)
def test_decode_shapes_agree(gpu, dev, tune, order):
    """Every split shape (pages per wave x waves per workgroup) gives the oracle's answer,
    with the fused and plain entries, on lengths that exercise 1..many splits, in every
    grid order (split-major, request-major, and the compact list of units with work)."""
    lens = [3, 64, 65, 500, 1023, 2048, 1500, 16]
    positions = [n - 1 for n in lens]
    tune(decode_order=order)
    for pages in ("1", "2", "4"):
        for waves in ("4", "8"):
            tune(decode_pages=pages, decode_waves=waves)
            k2, v2, k1, v1, o2, o1, q, tables = _fused_vs_separate(
                gpu, dev, lens, positions, 12, 3, seed=int(pages) * 10 + int(waves))
            assert np.array_equal(k2, k1) and np.array_equal(v2, v1)
            assert np.array_equal(o2.view(np.uint32), o1.view(np.uint32)), (pages, waves)
            want = _oracle(q.astype(np.float32), k1, v1, tables, lens, 12, 3, 3, 1)
            element_gate(o2, want, f"shape {pages} x {waves}, order {order}")


def test_grid_orders_are_bit_identical(gpu, dev, tune):
    """The grid order only places the workgroups: splits merge in split order whatever
    order they finish in, so every order gives the same bits."""
    lens = [1, 17, 256, 257, 700, 2048, 1999, 64, 0, 1024]
    positions = [max(n - 1, 0) for n in lens]
    outs = []
    for order in ORDERS:
        tune(decode_order=order)
        _, _, _, _, o2, o1, _, _ = _fused_vs_separate(gpu, dev, lens, positions, 12, 3, seed=5)
        assert np.array_equal(o2.view(np.uint32), o1.view(np.uint32))
        outs.append(o2.view(np.uint32))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


@pytest.mark.parametrize("batch", [64, 70, 256, 260])
def test_batch_at_and_past_the_compact_limit(gpu, dev, batch):
    """The compact order's search holds up to four requests per lane: 64 requests fill one
    set of lanes, 70 and 256 take two and four, and above 256 the launch falls back to the
    request-major grid. The answer is the oracle's either way, and inactive requests keep
    their output."""
    lens = [int(x) for x in np.random.default_rng(44 + batch).integers(0, 700, batch)]
    lens[3] = 0
    lens[batch - 1] = 0
    q, k_pool, v_pool, tables, stride = _case(45, lens, 12, 3)
    got = _run_decode(gpu, dev, q, k_pool, v_pool, tables, lens, 12, 3, 3, 1, stride * 16)
    want = _oracle(q, k_pool, v_pool, tables, lens, 12, 3, 3, 1)
    active = np.asarray(lens) > 0
    element_gate(got[active], want[active], f"batch {batch}")
    assert np.all(got[~active] == SENTINEL)


def test_workspace_shared_across_batch_sizes(gpu, dev):
    """One workspace (sized for the largest call) serves decode calls whose batch size and
    context bound change from call to call, as the engine's active count does step to step:
    the split count, and with it the place of every partial, moves between calls. Each launch
    leaves its combine counters back at zero."""
    rng = np.random.default_rng(90)
    n_head, n_kv, n_layer, max_batch, stride = 12, 3, 2, 16, 128
    nbytes = gpu.lib.crucible_attention_decode_workspace_bytes(max_batch, n_head, stride * 16)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    n_pages = max_batch * stride + 2
    kp, vp = random_pools(rng, n_pages, n_layer, n_kv * 64)
    d_k, d_v = _dev(kp, dev), _dev(vp, dev)
    for batch, max_seq in ((16, 2048), (5, 512), (11, 2048), (16, 1024), (1, 2048), (16, 2048),
                           (3, 256)):
        lens = rng.integers(1, max_seq + 1, batch)
        tables = disjoint_tables(rng, n_pages, lens, stride)
        q = rng.standard_normal((batch, n_head * 64)).astype(np.float16).astype(np.float32)
        out = torch.full((batch, n_head * 64), SENTINEL, device=dev)
        gpu.attention_decode_paged(_dev(q.astype(np.float16), dev), d_k, d_v, out,
                                   _dev(tables, dev), _dev(lens.astype(np.int32), dev), batch,
                                   n_head, n_kv, 64, stride, n_layer, 1, n_kv * 64, max_seq,
                                   workspace=ws)
        torch.cuda.synchronize()
        want = _oracle(q, kp, vp, tables, lens, n_head, n_kv, n_layer, 1)
        element_gate(out.cpu().numpy(), want, f"shared workspace, batch {batch}, max_seq {max_seq}")
        assert int(torch.count_nonzero(ws[:65536 * 4])) == 0, f"counters not reset, batch {batch}"


@pytest.mark.parametrize("n_head,n_kv,pad", [(12, 3, 0), (12, 12, 4), (16, 4, 0), (12, 1, 8)])
def test_qkv_rope_entry_equals_rope_split_then_fused_append(gpu, dev, n_head, n_kv, pad):
    """crucible_attention_decode_qkv_paged_append (q/k/v straight from the fused projection
    rows, RoPE in the same launch) gives the bytes of crucible_rope_split_qkv followed by
    crucible_attention_decode_paged_append: pools and outputs bit for bit, including an
    append off the last slot and an inactive request."""
    from crucible_amd.gpu_model import rope_tables

    rng = np.random.default_rng(n_head * 7 + n_kv + pad)
    lens = [1, 16, 17, 0, 300, 1024, 40]
    positions = [0, 15, 16, 5, 299, 1023, 100]
    batch, kv, n_layer, layer = len(lens), n_kv * 64, 3, 2
    stride = max(-(-max(max(lens), max(positions) + 1) // 16), 1)
    need = [max(-(-max(n, 1) // 16), (p >> 4) + 1) for n, p in zip(lens, positions)]
    n_pages = sum(need) + 3
    kp, vp = random_pools(rng, n_pages, n_layer, kv)
    tables = disjoint_tables(rng, n_pages, [16 * k for k in need], stride)
    width = (n_head + 2 * n_kv) * 64
    qkv = np.zeros((batch, width + pad), np.float32)
    qkv[:, :width] = rng.standard_normal((batch, width)).astype(np.float32)
    cos, sin = rope_tables(64, stride * 16, 10000.0)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    d_qkv, d_cos, d_sin = d(qkv), d(cos), d(sin)
    d_tab, d_pos, d_len = d(tables), d(np.asarray(positions, np.int32)), d(np.asarray(lens, np.int32))
    max_seq = stride * 16
    # reference order: split + rotate, then the fused append + decode
    q = torch.empty((batch, n_head * 64), device=dev)
    k = torch.empty((batch, kv), device=dev)
    v = torch.empty((batch, kv), device=dev)
    gpu.rope_split_qkv(d_qkv[:, :width].contiguous(), q, k, v, d_cos, d_sin, d_pos, n_head, n_kv)
    k1, v1 = _dev(kp, dev), _dev(vp, dev)
    out1 = torch.full((batch, n_head * 64), SENTINEL, device=dev)
    gpu.attention_decode_paged_append(q, k, v, k1, v1, out1, d_tab, d_pos, d_len, batch, n_head,
                                      n_kv, 64, stride, n_layer, layer, kv, max_seq)
    k2, v2 = _dev(kp, dev), _dev(vp, dev)
    out2 = torch.full((batch, n_head * 64), SENTINEL, device=dev)
    gpu.attention_decode_qkv_paged_append(d_qkv, d_cos, d_sin, k2, v2, out2, d_tab, d_pos, d_len,
                                          batch, n_head, n_kv, 64, stride, n_layer, layer, kv,
                                          max_seq)
    torch.cuda.synchronize()
    assert torch.equal(k1, k2) and torch.equal(v1, v2), "pool bytes differ"
    o1, o2 = out1.cpu().numpy(), out2.cpu().numpy()
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32)), "outputs differ"
    assert np.all(o2[3] == SENTINEL)
    # and against the oracle: rotate on the host (exact f32 ops), append, attend
    qr = qkv[:, :n_head * 64].reshape(batch, n_head, 64).copy()
    c = cos[positions][:, None, :]
    s = sin[positions][:, None, :]
    lo, hi = qr[..., :32].copy(), qr[..., 32:].copy()
    qr[..., :32], qr[..., 32:] = lo * c - hi * s, lo * s + hi * c
    want = _oracle(qr.reshape(batch, -1), k1.cpu().numpy().view(np.uint16),
                   v1.cpu().numpy().view(np.uint16), tables, lens, n_head, n_kv, n_layer, layer)
    active = [b for b, n in enumerate(lens) if n > 0]
    element_gate(o2[active], want[active], f"qkv entry {n_head}/{n_kv}")


def test_qkv_entry_without_rope_equals_plain_fused_append(gpu, dev):
    """With no rope tables the qkv entry is the fused append + decode on strided rows."""
    rng = np.random.default_rng(5)
    lens = [33, 200, 7]
    positions = [32, 199, 6]
    n_head, n_kv, batch, kv, n_layer, layer, stride = 12, 3, 3, 192, 2, 0, 16
    need = [-(-n // 16) for n in lens]
    n_pages = sum(need) + 2
    kp, vp = random_pools(rng, n_pages, n_layer, kv)
    tables = disjoint_tables(rng, n_pages, [16 * k for k in need], stride)
    width = (n_head + 2 * n_kv) * 64
    qkv = rng.standard_normal((batch, width)).astype(np.float32)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    d_tab, d_pos, d_len = d(tables), d(np.asarray(positions, np.int32)), d(np.asarray(lens, np.int32))
    k1, v1 = _dev(kp, dev), _dev(vp, dev)
    out1 = torch.full((batch, n_head * 64), SENTINEL, device=dev)
    gpu.attention_decode_paged_append(d(qkv[:, :768]), d(qkv[:, 768:960]), d(qkv[:, 960:]), k1, v1,
                                      out1, d_tab, d_pos, d_len, batch, n_head, n_kv, 64, stride,
                                      n_layer, layer, kv, stride * 16)
    k2, v2 = _dev(kp, dev), _dev(vp, dev)
    out2 = torch.full((batch, n_head * 64), SENTINEL, device=dev)
    gpu.attention_decode_qkv_paged_append(d(qkv), None, None, k2, v2, out2, d_tab, d_pos, d_len,
                                          batch, n_head, n_kv, 64, stride, n_layer, layer, kv,
                                          stride * 16)
    torch.cuda.synchronize()
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    assert torch.equal(out1, out2)


PLAN_OFFSET = 65536 * 4          # the unit plan follows the counters in the workspace
PLAN_ENTRY_INTS = 192


def test_unit_plan_reuse_equals_a_fresh_search(gpu, dev):
    """The compact order's unit plan: a launch whose lengths, positions and geometry equal
    the previous launch's takes its unit and page ids from the workspace instead of
    searching. Every call here runs twice, once on a warm workspace (whose plan the earlier
    calls left) and once on a fresh one (nothing planned): outputs and pools must agree bit
    for bit. The sequence covers a repeated call (planned), a table rewritten under equal
    lengths (the page-id check reloads the pages from the new ids, attended and
    append-only units), a changed length, changed append positions, the decode-only kernel
    on the fused kernel's plan and back, and a smaller batch."""
    rng = np.random.default_rng(2026)
    n_head, n_kv, n_layer, layer, stride = 12, 3, 2, 1, 128
    batch, max_seq, kv = 16, 2048, n_kv * 64
    n_pages = batch * stride + 64
    kp0, vp0 = random_pools(rng, n_pages, n_layer, kv)
    lens = rng.integers(64, max_seq, batch).astype(np.int32)
    tables = disjoint_tables(rng, n_pages, lens + 1, stride)
    q = _dev(rng.standard_normal((batch, n_head * 64)).astype(np.float16), dev)
    k_new = _dev(rng.standard_normal((batch, kv)).astype(np.float32), dev)
    v_new = _dev(rng.standard_normal((batch, kv)).astype(np.float32), dev)
    nbytes = gpu.lib.crucible_attention_decode_workspace_bytes(batch, n_head, max_seq)
    warm = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    pools = {"warm": (_dev(kp0, dev), _dev(vp0, dev)), "fresh": (_dev(kp0, dev), _dev(vp0, dev))}

    def run(tab, ln, pos, b=batch, fused=True):
        outs = {}
        for name in ("warm", "fresh"):
            ws = warm if name == "warm" else torch.zeros_like(warm)
            k, v = pools[name]
            out = torch.full((b, n_head * 64), SENTINEL, device=dev)
            args = (_dev(tab[:b], dev), _dev(pos[:b], dev), _dev(ln[:b], dev))
            if fused:
                gpu.attention_decode_paged_append(q[:b], k_new[:b], v_new[:b], k, v, out,
                                                  args[0], args[1], args[2], b, n_head, n_kv,
                                                  64, stride, n_layer, layer, kv, max_seq,
                                                  workspace=ws)
            else:
                gpu.attention_decode_paged(q[:b], k, v, out, args[0], args[2], b, n_head, n_kv,
                                           64, stride, n_layer, layer, kv, max_seq, workspace=ws)
            torch.cuda.synchronize()
            outs[name] = out.cpu()
        assert torch.equal(outs["warm"].view(torch.int32), outs["fresh"].view(torch.int32))
        for (kw, vw), (kf, vf) in [(pools["warm"], pools["fresh"])]:
            assert torch.equal(kw.view(torch.int16), kf.view(torch.int16))
            assert torch.equal(vw.view(torch.int16), vf.view(torch.int16))
        return outs["warm"]

    ln = lens + 1
    pos = lens.copy()
    first = run(tables, ln, pos)
    entry0 = warm[PLAN_OFFSET:PLAN_OFFSET + 4 * PLAN_ENTRY_INTS].view(torch.int32).cpu()
    assert int(entry0[0]) == 1 and int(entry0[1]) & 127 == batch  # the plan was written
    again = run(tables, ln, pos)
    assert torch.equal(first.view(torch.int32), again.view(torch.int32))
    # a rewritten table under equal lengths: request 3's pages move to unused pages (with
    # other contents), including the page its row is appended to
    used = set(int(x) for b in range(batch) for x in tables[b, :-(-int(ln[b]) // 16)])
    free = [p for p in range(n_pages) if p not in used]
    t2 = tables.copy()
    n3 = -(-int(ln[3]) // 16)
    t2[3, :n3] = free[:n3]
    run(t2, ln, pos)
    run(t2, ln, pos)
    # a changed length, then changed append positions under equal lengths
    ln2 = ln.copy()
    ln2[5] -= 17
    run(t2, ln2, pos)
    pos2 = pos.copy()
    pos2[7] = min(int(ln2[7]) + 300, stride * 16 - 1)  # past the attended keys' splits
    t2[7, pos2[7] // 16] = free[n3]                     # its page: an unused one
    run(t2, ln2, pos2)
    run(t2, ln2, pos2)
    # the decode-only kernel on the fused kernel's plan, then the fused kernel again
    run(t2, ln2, pos2, fused=False)
    run(t2, ln2, pos2)
    # a smaller batch on the same workspace
    run(t2, ln2, pos2, b=11)
    run(t2, ln2, pos2, b=11)


def test_unit_plan_with_the_qkv_rope_entry(gpu, dev):
    """The unit plan under the fused q/k/v entry (RoPE of q and k, both appends, decode; the
    compact order at config 3's shape): calls on a warm workspace (the plan of the previous
    call, then of the fused entry without RoPE, whose plan it shares) equal calls on a
    zeroed one, bit for bit."""
    from crucible_amd.gpu_model import rope_tables

    rng = np.random.default_rng(2027)
    n_head, n_kv, n_layer, layer, stride = 12, 3, 2, 0, 128
    batch, max_seq, kv = 16, 2048, n_kv * 64
    n_pages = batch * stride + 16
    kp0, vp0 = random_pools(rng, n_pages, n_layer, kv)
    lens = rng.integers(64, max_seq, batch).astype(np.int32)
    tables = disjoint_tables(rng, n_pages, lens, stride)
    width = (n_head + 2 * n_kv) * 64
    qkv = _dev(rng.standard_normal((batch, width)).astype(np.float32), dev)
    cos, sin = rope_tables(64, max_seq, 10000.0)
    d_cos, d_sin = _dev(cos, dev), _dev(sin, dev)
    d_tab, d_len, d_pos = _dev(tables, dev), _dev(lens, dev), _dev(lens - 1, dev)
    nbytes = gpu.lib.crucible_attention_decode_workspace_bytes(batch, n_head, max_seq)
    warm = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    pools = {"warm": (_dev(kp0, dev), _dev(vp0, dev)), "fresh": (_dev(kp0, dev), _dev(vp0, dev))}

    def run(rope=True):
        outs = {}
        for name in ("warm", "fresh"):
            ws = warm if name == "warm" else torch.zeros_like(warm)
            k, v = pools[name]
            out = torch.full((batch, n_head * 64), SENTINEL, device=dev)
            gpu.attention_decode_qkv_paged_append(qkv, d_cos if rope else None,
                                                  d_sin if rope else None, k, v, out, d_tab,
                                                  d_pos, d_len, batch, n_head, n_kv, 64, stride,
                                                  n_layer, layer, kv, max_seq, workspace=ws)
            torch.cuda.synchronize()
            outs[name] = out.cpu()
        assert torch.equal(outs["warm"].view(torch.int32), outs["fresh"].view(torch.int32))
        (kw, vw), (kf, vf) = pools["warm"], pools["fresh"]
        assert torch.equal(kw.view(torch.int16), kf.view(torch.int16))
        assert torch.equal(vw.view(torch.int16), vf.view(torch.int16))

    run()
    run()
    run(rope=False)
    run()


def test_unit_plan_is_not_taken_for_other_pools(gpu, dev):
    """A plan entry records the table and pool addresses it was made for: a call with equal
    lengths and shape on other pools and another table rebuilds it (its entries then hold
    the new addresses) and equals a call on a zeroed workspace, bit for bit; so does a call
    with the same table and other pools. Both pools have the same number of pages, so no
    page id of either table lies outside the other pool."""
    rng = np.random.default_rng(2028)
    n_head, n_kv, n_layer, layer, stride = 12, 3, 1, 0, 128
    batch, max_seq, kv = 16, 2048, n_kv * 64
    n_pages = batch * stride
    lens = rng.integers(64, max_seq, batch).astype(np.int32)
    q = _dev(rng.standard_normal((batch, n_head * 64)).astype(np.float16), dev)
    k_new = _dev(rng.standard_normal((batch, kv)).astype(np.float32), dev)
    v_new = _dev(rng.standard_normal((batch, kv)).astype(np.float32), dev)
    d_len, d_pos = _dev(lens, dev), _dev(lens - 1, dev)
    nbytes = gpu.lib.crucible_attention_decode_workspace_bytes(batch, n_head, max_seq)
    warm = torch.zeros(nbytes, dtype=torch.uint8, device=dev)

    def call(ws, k, v, tab):
        out = torch.full((batch, n_head * 64), SENTINEL, device=dev)
        gpu.attention_decode_paged_append(q, k_new, v_new, k, v, out, tab, d_pos, d_len, batch,
                                          n_head, n_kv, 64, stride, n_layer, layer, kv, max_seq,
                                          workspace=ws)
        torch.cuda.synchronize()
        return out.cpu()

    pools = []
    for _ in range(2):
        kp, vp = random_pools(rng, n_pages, n_layer, kv)
        pools.append((_dev(kp, dev), _dev(vp, dev), _dev(disjoint_tables(rng, n_pages, lens, stride), dev)))
    ka, va, ta = pools[0]
    kb, vb, tb = pools[1]
    call(warm, ka, va, ta)
    kb2, vb2 = kb.clone(), vb.clone()
    got = call(warm, kb, vb, tb)
    want = call(torch.zeros_like(warm), kb2, vb2, tb)
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))
    assert torch.equal(kb.view(torch.int16), kb2.view(torch.int16))

    def addresses():
        # the entry's words 6..11: the table, k_pool and v_pool addresses it was made for
        e = warm[PLAN_OFFSET:PLAN_OFFSET + 4 * PLAN_ENTRY_INTS].view(torch.int32).cpu().numpy()
        w = [int(x) & 0xFFFFFFFF for x in e[6:12]]
        return [w[0] | w[1] << 32, w[2] | w[3] << 32, w[4] | w[5] << 32]

    assert addresses() == [tb.data_ptr(), kb.data_ptr(), vb.data_ptr()]
    # the same table address with the other pools: the entry is rebuilt for those pools
    call(warm, ka, va, ta)
    assert addresses() == [ta.data_ptr(), ka.data_ptr(), va.data_ptr()]
    kc, vc = kb.clone(), vb.clone()
    got = call(warm, kb, vb, ta)
    assert addresses() == [ta.data_ptr(), kb.data_ptr(), vb.data_ptr()]
    want = call(torch.zeros_like(warm), kc, vc, ta)
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))
    assert torch.equal(kb.view(torch.int16), kc.view(torch.int16))
    assert torch.equal(vb.view(torch.int16), vc.view(torch.int16))


def test_cached_workspace_is_zeroed_when_the_pools_change(gpu, dev):
    """Gpu.workspace keeps one workspace per shape and zeroes it when a call brings other
    pools (address or size), so a plan made for one pool never meets a pool reallocated
    smaller at the same address."""
    batch, n_head, max_seq = 4, 12, 512
    k1 = torch.zeros(4096, dtype=torch.float16, device=dev)
    v1 = torch.zeros(4096, dtype=torch.float16, device=dev)
    ws = gpu.workspace(batch, n_head, max_seq, (k1, v1))
    ws[PLAN_OFFSET:PLAN_OFFSET + 64].fill_(7)
    assert gpu.workspace(batch, n_head, max_seq, (k1, v1)) is ws
    assert int(ws[PLAN_OFFSET:PLAN_OFFSET + 64].sum()) == 7 * 64  # same pools: kept
    assert gpu.workspace(batch, n_head, max_seq, (k1[:2048], v1[:2048])) is ws
    assert int(ws.sum()) == 0  # same addresses, fewer elements: zeroed
    ws[PLAN_OFFSET:PLAN_OFFSET + 64].fill_(7)
    k2 = torch.zeros(4096, dtype=torch.float16, device=dev)
    gpu.workspace(batch, n_head, max_seq, (k2, v1[:2048]))
    assert int(ws.sum()) == 0  # another address: zeroed


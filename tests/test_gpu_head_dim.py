"""head_dim other than 64.

The reference kernels take any head_dim (kernels.cu:1741-1756 decode, 2100-2276 prefill:
loops over d). The library runs head_dim 64 on its MFMA kernels and any other multiple of 8
up to 256 on the generic kernels (generic_attend.hpp). Every decode and prefill entry point
is checked here against the f64 oracle under the reference's element gate
(|d| <= 2e-5 + 2e-5 |ref|, gpu_attention_validation.rs:20-22) and the north-star 2e-3; the
fused entries must store the same pool bytes and give the same output bits as their separate
calls, slots past a request's end must not be read (NaN there changes nothing), inactive
requests keep their output, and the hybrid segment form equals the pool path.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from attn_cases import disjoint_tables, random_pools
from crucible_amd import _lib
from gates import element_gate

pytestmark = pytest.mark.gpu

SENTINEL = -12345.25
HDS = [32, 96, 128, 256]
NAN16 = np.uint16(0x7E00)


def _dev(a, dev):
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.float16).copy()).to(dev)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _heads(hd):
    # fewer heads at the widest dimension keeps the oracle fast
    return (8, 2) if hd >= 128 else (12, 3)


def _decode_case(seed, hd, lens, n_layer=2):
    rng = np.random.default_rng(seed)
    n_head, n_kv = _heads(hd)
    stride = max(1, -(-max(max(lens), 1) // 16))
    n_pages = sum(-(-max(n, 1) // 16) for n in lens) + 4
    kp, vp = random_pools(rng, n_pages, n_layer, n_kv * hd)
    tables = disjoint_tables(rng, n_pages, [max(n, 1) for n in lens], stride)
    q = rng.standard_normal((len(lens), n_head * hd)).astype(np.float32)
    return rng, n_head, n_kv, stride, n_pages, kp, vp, tables, q


def _poison_past_the_end(kp, vp, tables, lens, n_layer, layer, kv):
    """NaN into every slot of a request's last page at or past its length (K rows and V^T
    columns of this layer)."""
    kp, vp = kp.copy(), vp.copy()
    for b, n in enumerate(lens):
        if n <= 0 or n % 16 == 0:
            continue
        page = int(tables[b, (n - 1) // 16])
        base = (page * n_layer + layer) * 16 * kv
        for slot in range(n % 16, 16):
            kp[base + slot * kv: base + (slot + 1) * kv] = NAN16
            vp[base + slot: base + 16 * kv: 16] = NAN16
    return kp, vp


@pytest.mark.parametrize("hd", HDS)
@pytest.mark.parametrize("q_dtype,out_dtype", [(torch.float16, torch.float32),
                                               (torch.float32, torch.float16)])
def test_decode_paged_matches_oracle(gpu, dev, hd, q_dtype, out_dtype):
    lens = [1, 15, 16, 17, 64, 65, 129, 0, 700, 1024]
    n_layer, layer = 2, 1
    rng, n_head, n_kv, stride, _, kp, vp, tables, q = _decode_case(hd, hd, lens, n_layer)
    if q_dtype == torch.float16:
        q = q.astype(np.float16).astype(np.float32)
    kv = n_kv * hd
    d_lens = _dev(np.asarray(lens, np.int32), dev)
    outs = []
    for k_host, v_host in [(kp, vp), _poison_past_the_end(kp, vp, tables, lens, n_layer, layer, kv)]:
        out = torch.full((len(lens), n_head * hd), SENTINEL, dtype=out_dtype, device=dev)
        gpu.attention_decode_paged(torch.from_numpy(q).to(dev).to(q_dtype), _dev(k_host, dev),
                                   _dev(v_host, dev), out, _dev(tables, dev), d_lens, len(lens),
                                   n_head, n_kv, hd, stride, n_layer, layer, kv, stride * 16)
        torch.cuda.synchronize()
        outs.append(out.float().cpu().numpy())
    got = outs[0]
    assert np.array_equal(got.view(np.uint32), outs[1].view(np.uint32)), "slots past the end read"
    active = [b for b, n in enumerate(lens) if n > 0]
    sentinel = np.float32(np.float16(SENTINEL)) if out_dtype == torch.float16 else SENTINEL
    assert np.all(got[[b for b, n in enumerate(lens) if n <= 0]] == np.float32(sentinel))
    want = oracle.attention_paged_rows(q[active], kp, vp, tables[active],
                                       np.asarray([lens[b] for b in active], np.int32),
                                       n_head=n_head, n_kv_head=n_kv, head_dim=hd,
                                       table_stride=stride, n_layer=n_layer, layer=layer)
    element_gate(got[active], want, f"decode hd {hd}", out_f16=out_dtype == torch.float16)


@pytest.mark.parametrize("hd", HDS)
@pytest.mark.parametrize("kv_dtype", [torch.float32, torch.float16])
def test_fused_append_decode_equals_separate_calls(gpu, dev, hd, kv_dtype):
    lens = [1, 16, 17, 300, 1000, 0]
    positions = [max(n - 1, -1) for n in lens]
    n_layer, layer = 2, 0
    rng, n_head, n_kv, stride, _, kp, vp, tables, q = _decode_case(7 + hd, hd, lens, n_layer)
    kv = n_kv * hd
    k_new = rng.standard_normal((len(lens), kv)).astype(np.float32)
    v_new = rng.standard_normal((len(lens), kv)).astype(np.float32)
    d_q = torch.from_numpy(q).to(dev)
    d_tables, d_pos = _dev(tables, dev), _dev(np.asarray(positions, np.int32), dev)
    d_lens = _dev(np.asarray(lens, np.int32), dev)
    d_kn, d_vn = (torch.from_numpy(x).to(dev).to(kv_dtype) for x in (k_new, v_new))
    # separate calls: two appends, then decode
    k1, v1 = _dev(kp, dev), _dev(vp, dev)
    gpu.cache_store_rows_paged(d_kn, k1, d_tables, d_pos, len(lens), kv, stride, n_layer, layer,
                               kind="k")
    gpu.cache_store_rows_paged(d_vn, v1, d_tables, d_pos, len(lens), kv, stride, n_layer, layer,
                               kind="v")
    o1 = torch.full((len(lens), n_head * hd), SENTINEL, device=dev)
    gpu.attention_decode_paged(d_q, k1, v1, o1, d_tables, d_lens, len(lens), n_head, n_kv, hd,
                               stride, n_layer, layer, kv, stride * 16)
    # fused entry, and its allocation-free twin
    for entry in ("workspace", "noalloc"):
        k2, v2 = _dev(kp, dev), _dev(vp, dev)
        o2 = torch.full_like(o1, SENTINEL)
        args = (d_q, d_kn, d_vn, k2, v2, o2, d_tables, d_pos, d_lens, len(lens), n_head, n_kv,
                hd, stride, n_layer, layer, kv, stride * 16)
        if entry == "workspace":
            gpu.attention_decode_paged_append(*args)
        else:
            _lib.check(gpu.lib.crucible_attention_decode_paged_append_noalloc(
                d_q.data_ptr(), _lib.F32, d_kn.data_ptr(), d_vn.data_ptr(),
                _lib.F16 if kv_dtype == torch.float16 else _lib.F32, k2.data_ptr(),
                v2.data_ptr(), o2.data_ptr(), _lib.F32, d_tables.data_ptr(), d_pos.data_ptr(),
                d_lens.data_ptr(), len(lens), n_head, n_kv, hd, stride, n_layer, layer, kv,
                stride * 16, ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))
        torch.cuda.synchronize()
        assert torch.equal(k1, k2) and torch.equal(v1, v2), f"{entry}: pool bytes differ"
        assert torch.equal(o1, o2), f"{entry}: outputs differ"
    active = [b for b, n in enumerate(lens) if n > 0]
    k_host = k1.cpu().numpy().view(np.uint16)
    v_host = v1.cpu().numpy().view(np.uint16)
    want = oracle.attention_paged_rows(q[active], k_host, v_host, tables[active],
                                       np.asarray([lens[b] for b in active], np.int32),
                                       n_head=n_head, n_kv_head=n_kv, head_dim=hd,
                                       table_stride=stride, n_layer=n_layer, layer=layer)
    element_gate(o1.cpu().numpy()[active], want, f"fused hd {hd}")


@pytest.mark.parametrize("hd", HDS)
@pytest.mark.parametrize("rope", [True, False])
def test_qkv_entry_equals_rope_split_then_fused_append(gpu, dev, hd, rope):
    lens = [5, 64, 333, 1024]
    positions = [n - 1 for n in lens]
    n_layer, layer = 2, 1
    rng, n_head, n_kv, stride, _, kp, vp, tables, _ = _decode_case(11 + hd, hd, lens, n_layer)
    kv = n_kv * hd
    ld = n_head * hd + 2 * kv + 8  # padded rows
    qkv = rng.standard_normal((len(lens), ld)).astype(np.float32)
    cos_t, sin_t = oracle.rope_table(hd, stride * 16)
    d_qkv = _dev(qkv, dev)
    d_cos, d_sin = (_dev(cos_t, dev), _dev(sin_t, dev)) if rope else (None, None)
    d_tables, d_pos = _dev(tables, dev), _dev(np.asarray(positions, np.int32), dev)
    d_lens = _dev(np.asarray(lens, np.int32), dev)
    # the separate path: rope split (or a plain split), then the fused append + decode
    q = torch.empty((len(lens), n_head * hd), device=dev)
    k = torch.empty((len(lens), kv), device=dev)
    v = torch.empty((len(lens), kv), device=dev)
    if rope:
        gpu.rope_split_qkv(d_qkv, q, k, v, d_cos, d_sin, d_pos, n_head, n_kv, head_dim=hd)
    else:
        q.copy_(d_qkv[:, :n_head * hd])
        k.copy_(d_qkv[:, n_head * hd:n_head * hd + kv])
        v.copy_(d_qkv[:, n_head * hd + kv:n_head * hd + 2 * kv])
    k1, v1 = _dev(kp, dev), _dev(vp, dev)
    o1 = torch.full((len(lens), n_head * hd), SENTINEL, device=dev)
    gpu.attention_decode_paged_append(q, k, v, k1, v1, o1, d_tables, d_pos, d_lens, len(lens),
                                      n_head, n_kv, hd, stride, n_layer, layer, kv, stride * 16)
    k2, v2 = _dev(kp, dev), _dev(vp, dev)
    o2 = torch.full_like(o1, SENTINEL)
    gpu.attention_decode_qkv_paged_append(d_qkv, d_cos, d_sin, k2, v2, o2, d_tables, d_pos,
                                          d_lens, len(lens), n_head, n_kv, hd, stride, n_layer,
                                          layer, kv, stride * 16)
    torch.cuda.synchronize()
    assert torch.equal(k1, k2) and torch.equal(v1, v2), "pool bytes differ"
    assert torch.equal(o1, o2), "outputs differ"
    # the rotation itself against the oracle's RopeTable::apply
    if rope:
        qh = q.cpu().numpy()
        for b in (0, len(lens) - 1):
            for h in (0, n_head - 1):
                raw = qkv[b, h * hd:(h + 1) * hd]
                assert np.array_equal(qh[b, h * hd:(h + 1) * hd],
                                      oracle.rope_apply(raw, cos_t, sin_t, positions[b]))
    k_host = k2.cpu().numpy().view(np.uint16)
    v_host = v2.cpu().numpy().view(np.uint16)
    want = oracle.attention_paged_rows(q.cpu().numpy(), k_host, v_host, tables,
                                       np.asarray(lens, np.int32), n_head=n_head, n_kv_head=n_kv,
                                       head_dim=hd, table_stride=stride, n_layer=n_layer,
                                       layer=layer)
    element_gate(o2.cpu().numpy(), want, f"qkv hd {hd} rope {rope}")


@pytest.mark.parametrize("hd", HDS)
def test_contiguous_decode_and_split_forms(gpu, dev, hd):
    """The contiguous cache ([layer][cap/16] 16-token blocks, the pool layout with page =
    position >> 4) through attention_decode and attention_split, against the paged entry on
    the same blocks (same kernel: bit-identical) and the oracle."""
    rng = np.random.default_rng(3 + hd)
    n_head, n_kv = _heads(hd)
    kv, cap, n_layer, layer = n_kv * hd, 512, 2, 1
    k_c, v_c = random_pools(rng, cap // 16, n_layer, kv)
    # the same memory as a pool whose page p of layer `layer` is block p of the layer region
    for length in (1, 17, 128, 511):
        q = rng.standard_normal((1, n_head * hd)).astype(np.float32)
        params = _dev(np.array([0, 0, length - 1, length, 0, 0], np.int32), dev)
        d_q, d_k, d_v = _dev(q, dev), _dev(k_c, dev), _dev(v_c, dev)
        out_c = torch.full((1, n_head * hd), SENTINEL, device=dev)
        gpu.attention_decode(d_q, d_k, d_v, out_c, n_head, n_kv, hd, params, cap, kv,
                             layer * cap * kv)
        n_chunks = -(-cap // 128)
        po = torch.full((n_head * n_chunks * hd,), SENTINEL, device=dev)
        pm = torch.full((n_head * n_chunks,), SENTINEL, device=dev)
        pl = torch.full((n_head * n_chunks,), SENTINEL, device=dev)
        out_s = torch.full_like(out_c, SENTINEL)
        gpu.attention_split(d_q, d_k, d_v, po, pm, pl, out_s, n_head, n_kv, hd, params, cap, kv,
                            layer * cap * kv)
        # paged view: table = identity over the layer's blocks, n_layer 1 at that offset
        k_layer = k_c[layer * cap * kv:(layer + 1) * cap * kv]
        v_layer = v_c[layer * cap * kv:(layer + 1) * cap * kv]
        table = np.arange(cap // 16, dtype=np.int32)[None]
        out_p = torch.full_like(out_c, SENTINEL)
        gpu.attention_decode_paged(d_q, _dev(k_layer, dev), _dev(v_layer, dev), out_p,
                                   _dev(table, dev), _dev(np.array([length], np.int32), dev), 1,
                                   n_head, n_kv, hd, cap // 16, 1, 0, kv, cap)
        torch.cuda.synchronize()
        assert torch.equal(out_c, out_p) and torch.equal(out_c, out_s), length
        want = oracle.attention_paged_rows(q, k_layer, v_layer, table,
                                           np.array([length], np.int32), n_head=n_head,
                                           n_kv_head=n_kv, head_dim=hd, table_stride=cap // 16,
                                           n_layer=1, layer=0)
        element_gate(out_c.cpu().numpy(), want, f"contiguous hd {hd} len {length}")


def _prefill_case(seed, hd, lens, starts, n_layer=2):
    """Packed prompt rows of several requests: request i holds rows for positions
    starts[i] .. starts[i] + lens[i] - 1 (its earlier keys are already in the pool)."""
    rng = np.random.default_rng(seed)
    n_head, n_kv = _heads(hd)
    kv = n_kv * hd
    total = [s + n for s, n in zip(starts, lens)]
    stride = -(-max(total) // 16)
    n_pages = sum(-(-t // 16) for t in total) + 2
    kp, vp = random_pools(rng, n_pages, n_layer, kv)
    tables = disjoint_tables(rng, n_pages, total, stride)
    rows = sum(lens)
    q = rng.standard_normal((rows, n_head * hd)).astype(np.float32)
    owners = np.concatenate([np.full(n, i, np.int32) for i, n in enumerate(lens)])
    positions = np.concatenate([np.arange(s, s + n, dtype=np.int32) for s, n in zip(starts, lens)])
    packed_start = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)
    segments = np.stack([packed_start, np.asarray(lens, np.int32), np.asarray(starts, np.int32),
                         np.arange(len(lens), dtype=np.int32)], 1).astype(np.int32)
    return rng, n_head, n_kv, kv, stride, kp, vp, tables, q, owners, positions, segments


@pytest.mark.parametrize("hd", HDS)
def test_prefill_segment_and_owner_forms_match_oracle(gpu, dev, hd):
    lens, starts = [1, 17, 40, 100], [0, 5, 16, 30]
    n_layer, layer = 2, 1
    (_, n_head, n_kv, kv, stride, kp, vp, tables, q, owners, positions,
     segments) = _prefill_case(5 + hd, hd, lens, starts, n_layer)
    rows = q.shape[0]
    d_q, d_k, d_v, d_t = _dev(q, dev), _dev(kp, dev), _dev(vp, dev), _dev(tables, dev)
    out_s = torch.full((rows + 1, n_head * hd), SENTINEL, device=dev)
    gpu.attention_prefill_tiled(d_q, d_k, d_v, None, None, out_s, d_t, _dev(segments, dev),
                                len(lens), max(lens), stride, n_head, n_kv, hd, n_layer, layer,
                                kv)
    out_o = torch.full_like(out_s, SENTINEL)
    gpu.attention_prefill_packed(d_q, d_k, d_v, out_o, d_t, _dev(owners, dev),
                                 _dev(positions, dev), rows, stride, n_head, n_kv, hd, n_layer,
                                 layer, kv, stride * 16)
    torch.cuda.synchronize()
    got = out_s.cpu().numpy()
    assert np.all(got[rows] == np.float32(SENTINEL)), "row past the last one written"
    assert torch.equal(out_s, out_o), "segment and owner forms differ"
    want = oracle.attention_paged_rows(q, kp, vp, tables, positions + 1, table_index=owners,
                                       n_head=n_head, n_kv_head=n_kv, head_dim=hd,
                                       table_stride=stride, n_layer=n_layer, layer=layer)
    element_gate(got[:rows], want, f"prefill hd {hd}")


@pytest.mark.parametrize("hd", HDS)
def test_prefill_params_and_contiguous_forms(gpu, dev, hd):
    """One sequence: params form (rows at params[5] + r through one table) and the
    contiguous cache, against the oracle and each other."""
    rng = np.random.default_rng(9 + hd)
    n_head, n_kv = _heads(hd)
    kv, cap, n_layer, layer = n_kv * hd, 256, 2, 0
    start, rows = 37, 150
    k_c, v_c = random_pools(rng, cap // 16, n_layer, kv)
    q = rng.standard_normal((rows, n_head * hd)).astype(np.float32)
    d_q = _dev(q, dev)
    out_c = torch.full((rows, n_head * hd), SENTINEL, device=dev)
    gpu.attention_prefill(d_q, _dev(k_c, dev), _dev(v_c, dev), out_c, rows, n_head, n_kv, hd,
                          cap, kv, layer * cap * kv, start)
    k_layer = k_c[layer * cap * kv:(layer + 1) * cap * kv]
    v_layer = v_c[layer * cap * kv:(layer + 1) * cap * kv]
    table = np.arange(cap // 16, dtype=np.int32)
    params = _dev(np.array([0, 0, 0, 0, 0, start], np.int32), dev)
    out_p = torch.full_like(out_c, SENTINEL)
    gpu.attention_prefill_paged(d_q, _dev(k_layer, dev), _dev(v_layer, dev), out_p,
                                _dev(table, dev), rows, n_head, n_kv, hd, 1, 0, kv, cap, params)
    torch.cuda.synchronize()
    assert torch.equal(out_c, out_p)
    pos = np.arange(start, start + rows, dtype=np.int32)
    want = oracle.attention_paged_rows(q, k_layer, v_layer, table[None], pos + 1,
                                       table_index=np.zeros(rows, np.int32), n_head=n_head,
                                       n_kv_head=n_kv, head_dim=hd, table_stride=cap // 16,
                                       n_layer=1, layer=0)
    element_gate(out_c.cpu().numpy(), want, f"params/contiguous hd {hd}")


@pytest.mark.parametrize("hd", HDS)
def test_hybrid_segments_equal_the_pool_path(gpu, dev, hd):
    """Hybrid tiled prefill (gpu.rs:1691-1697): the chunk's own keys come from current_k /
    current_v (f32, rounded to fp16 as the append stores them); with the pool's chunk slots
    poisoned the output equals the library's packed append followed by the pool path."""
    lens, starts = [9, 33, 70], [0, 20, 3]
    n_layer, layer = 2, 0
    (rng, n_head, n_kv, kv, stride, kp, vp, tables, q, owners, positions,
     segments) = _prefill_case(13 + hd, hd, lens, starts, n_layer)
    rows = q.shape[0]
    cur_k = rng.standard_normal((rows, kv)).astype(np.float32)
    cur_v = rng.standard_normal((rows, kv)).astype(np.float32)
    d_q, d_t = _dev(q, dev), _dev(tables, dev)
    d_own, d_pos = _dev(owners, dev), _dev(positions, dev)
    # pool path: append the chunk's rows, then attend from the pool
    k1, v1 = _dev(kp, dev), _dev(vp, dev)
    for src, pool, kind in ((cur_k, k1, "k"), (cur_v, v1, "v")):
        gpu.cache_store_packed_paged(_dev(src, dev), pool, d_t, d_own, d_pos, rows, kv, stride,
                                     n_layer, layer, kind=kind)
    o1 = torch.full((rows, n_head * hd), SENTINEL, device=dev)
    gpu.attention_prefill_tiled(d_q, k1, v1, None, None, o1, d_t, _dev(segments, dev),
                                len(lens), max(lens), stride, n_head, n_kv, hd, n_layer, layer, kv)
    # hybrid on a pool whose chunk slots hold NaN
    kp2, vp2 = kp.copy(), vp.copy()
    for r in range(rows):
        page = int(tables[owners[r], positions[r] // 16])
        base = (page * n_layer + layer) * 16 * kv
        slot = int(positions[r] % 16)
        kp2[base + slot * kv: base + (slot + 1) * kv] = NAN16
        vp2[base + slot: base + 16 * kv: 16] = NAN16
    o2 = torch.full_like(o1, SENTINEL)
    gpu.attention_prefill_tiled(d_q, _dev(kp2, dev), _dev(vp2, dev), _dev(cur_k, dev),
                                _dev(cur_v, dev), o2, d_t, _dev(segments, dev), len(lens),
                                max(lens), stride, n_head, n_kv, hd, n_layer, layer, kv,
                                hybrid=True)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    want = oracle.attention_paged_rows(q, k1.cpu().numpy().view(np.uint16),
                                       v1.cpu().numpy().view(np.uint16), tables, positions + 1,
                                       table_index=owners, n_head=n_head, n_kv_head=n_kv,
                                       head_dim=hd, table_stride=stride, n_layer=n_layer,
                                       layer=layer)
    element_gate(o1.cpu().numpy(), want, f"hybrid hd {hd}")

"""The allocation-free fused decode (crucible_attention_decode_paged_append_noalloc) against
the workspace form it shares its kernels with: same pool bytes and same output bits, on two
calls in a row (the second smaller, so the shared device scratch holds the first call's
partials when it starts), and both within the north-star bar of the f64 oracle."""
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


def _dev(a, dev):
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.float16).copy()).to(dev)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _case(seed, lens, n_head, n_kv, n_layer, stride):
    rng = np.random.default_rng(seed)
    kv = n_kv * 64
    need = [-(-n // 16) for n in lens]
    n_pages = sum(need) + 5
    kp, vp = random_pools(rng, n_pages, n_layer, kv)
    tables = disjoint_tables(rng, n_pages, lens, stride)
    q = rng.standard_normal((len(lens), n_head * 64)).astype(np.float16)
    k_new = (rng.standard_normal((len(lens), kv)) * 2).astype(np.float32)
    v_new = (rng.standard_normal((len(lens), kv)) * 2).astype(np.float32)
    return kp, vp, tables, q, k_new, v_new


def _call(lib, entry, dev, kp, vp, tables, q, k_new, v_new, lens, n_head, n_kv, n_layer, layer,
          stride, workspace=None, max_seq=None):
    """One launch through the C ABI on copies of the pools; returns (k, v, out) on the host."""
    batch = len(lens)
    kv = n_kv * 64
    d_k, d_v = _dev(kp, dev), _dev(vp, dev)
    d_q, d_kn, d_vn = _dev(q, dev), _dev(k_new, dev), _dev(v_new, dev)
    d_tab = _dev(tables, dev)
    d_len = _dev(np.asarray(lens, np.int32), dev)
    d_pos = _dev(np.asarray(lens, np.int32) - 1, dev)
    out = torch.full((batch, n_head * 64), SENTINEL, dtype=torch.float32, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    args = [d_q.data_ptr(), _lib.F16, d_kn.data_ptr(), d_vn.data_ptr(), _lib.F32,
            d_k.data_ptr(), d_v.data_ptr(), out.data_ptr(), _lib.F32, d_tab.data_ptr(),
            d_pos.data_ptr(), d_len.data_ptr(), batch, n_head, n_kv, 64, stride, n_layer, layer,
            kv, max_seq or stride * 16]
    if workspace is not None:
        args += [workspace.data_ptr(), workspace.numel()]
    _lib.check(entry(*args, stream))
    torch.cuda.synchronize(dev)
    return (d_k.cpu().numpy().view(np.uint16), d_v.cpu().numpy().view(np.uint16),
            out.cpu().numpy())


def test_noalloc_equals_workspace_form_on_two_calls(dev):
    lib = _lib.load()
    n_head, n_kv, n_layer, layer = 12, 3, 3, 2
    calls = [
        # config-3 shaped: 16 requests up to 2048 tokens (many splits per request)
        (np.random.default_rng(5).integers(64, 2048, 16).astype(int).tolist(), 128),
        # smaller: 5 requests, 512-token table
        ([300, 17, 512, 129, 64], 32),
    ]
    for i, (lens, stride) in enumerate(calls):
        print(f"no-alloc call {i}: batch {len(lens)}, max_seq {stride * 16}", flush=True)
        kp, vp, tables, q, k_new, v_new = _case(90 + i, lens, n_head, n_kv, n_layer, stride)
        nbytes = lib.crucible_attention_decode_workspace_bytes(len(lens), n_head, stride * 16)
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        k1, v1, o1 = _call(lib, lib.crucible_attention_decode_paged_append, dev, kp, vp, tables,
                           q, k_new, v_new, lens, n_head, n_kv, n_layer, layer, stride, ws)
        k2, v2, o2 = _call(lib, lib.crucible_attention_decode_paged_append_noalloc, dev, kp, vp,
                           tables, q, k_new, v_new, lens, n_head, n_kv, n_layer, layer, stride)
        assert np.array_equal(k2, k1) and np.array_equal(v2, v1), f"call {i}: pool bytes differ"
        assert np.array_equal(o2.view(np.uint32), o1.view(np.uint32)), f"call {i}: outputs differ"
        want = oracle.attention_paged_rows(q.astype(np.float32), k2, v2, tables,
                                           np.asarray(lens, np.int32), n_head=n_head,
                                           n_kv_head=n_kv, head_dim=64, table_stride=stride,
                                           n_layer=n_layer, layer=layer)
        err = element_gate(o2, want, f"no-alloc call {i}")
        print(f"no-alloc call {i}: max-abs {err:.3e} against the oracle", flush=True)


def test_noalloc_at_the_documented_limit(dev):
    """The header's limit for batch 16 x 12 query heads: max_seq 20,992 tokens (82 splits of
    16 pages) runs, bit-identical to the workspace form and within the element gate, with one
    request at the full length; max_seq 21,008 (83 splits) is refused before any launch."""
    lib = _lib.load()
    n_head, n_kv, n_layer, layer = 12, 3, 1, 0
    limit = 20992
    stride = limit // 16
    lens = [limit] + np.random.default_rng(7).integers(64, 1500, 15).astype(int).tolist()
    print(f"no-alloc limit: batch 16, max_seq {limit}", flush=True)
    kp, vp, tables, q, k_new, v_new = _case(77, lens, n_head, n_kv, n_layer, stride)
    nbytes = lib.crucible_attention_decode_workspace_bytes(len(lens), n_head, limit)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    k1, v1, o1 = _call(lib, lib.crucible_attention_decode_paged_append, dev, kp, vp, tables, q,
                       k_new, v_new, lens, n_head, n_kv, n_layer, layer, stride, ws)
    k2, v2, o2 = _call(lib, lib.crucible_attention_decode_paged_append_noalloc, dev, kp, vp,
                       tables, q, k_new, v_new, lens, n_head, n_kv, n_layer, layer, stride)
    assert np.array_equal(k2, k1) and np.array_equal(v2, v1)
    assert np.array_equal(o2.view(np.uint32), o1.view(np.uint32))
    want = oracle.attention_paged_rows(q.astype(np.float32), k2, v2, tables,
                                       np.asarray(lens, np.int32), n_head=n_head, n_kv_head=n_kv,
                                       head_dim=64, table_stride=stride, n_layer=n_layer,
                                       layer=layer)
    err = element_gate(o2, want, "no-alloc at the limit")
    print(f"no-alloc limit: max-abs {err:.3e}", flush=True)
    # one page more: 83 splits, refused (the same real buffers; nothing is launched)
    stride2 = stride + 1
    tab2 = np.zeros((16, stride2), np.int32)
    tab2[:, :stride] = tables
    d = {name: _dev(a, dev) for name, a in (("q", q), ("kn", k_new), ("vn", v_new), ("k", kp),
                                            ("v", vp), ("t", tab2))}
    d_len = _dev(np.asarray(lens, np.int32), dev)
    d_pos = _dev(np.asarray(lens, np.int32) - 1, dev)
    out = torch.zeros((16, n_head * 64), device=dev)
    rc = lib.crucible_attention_decode_paged_append_noalloc(
        d["q"].data_ptr(), _lib.F16, d["kn"].data_ptr(), d["vn"].data_ptr(), _lib.F32,
        d["k"].data_ptr(), d["v"].data_ptr(), out.data_ptr(), _lib.F32, d["t"].data_ptr(),
        d_pos.data_ptr(), d_len.data_ptr(), 16, n_head, n_kv, 64, stride2, n_layer, layer,
        n_kv * 64, limit + 16, None)
    assert rc == _lib.ERR_WORKSPACE and "static scratch" in _lib.last_error()[1]


def test_noalloc_rejects_calls_past_the_scratch(dev):
    """A call whose partials exceed the static scratch is refused before any launch."""
    lib = _lib.load()
    batch, n_head, n_kv, stride = 64, 16, 16, 4096  # 64 x 16 heads at 65536 tokens
    null = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rc = lib.crucible_attention_decode_paged_append_noalloc(
        null, _lib.F16, null, null, _lib.F32, null, null, null, _lib.F32, null, null, null,
        batch, n_head, n_kv, 64, stride, 1, 0, n_kv * 64, stride * 16, None)
    assert rc == _lib.ERR_WORKSPACE
    assert "static scratch" in _lib.last_error()[1]

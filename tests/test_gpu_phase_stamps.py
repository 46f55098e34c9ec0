"""The stamped diagnostic twin computes what the product library computes, and its stamps
are ordered.

libcrucible_attn_stamps.so is the product library with the decode source built with
-DCRUCIBLE_STAMPS; bench.py --phases reads its stamps to split a config-3 launch into
phases. Both libraries are loaded side by side here (separate ctypes handles) and run the
same fused append + decode of a config-3-sized batch (the compact grid order, multi-split
units with the in-kernel combine): outputs and pools must agree bit for bit, and every
attending workgroup's stamps must run forward through its phases.
"""
import ctypes
import os

import numpy as np
import pytest
import torch

from crucible_amd import _build, _lib
from crucible_amd.gpu import Gpu, pool_elems

pytestmark = pytest.mark.gpu


def _twin_gpu():
    lib = ctypes.CDLL(_build.STAMPS_LIB_PATH)
    for name, (args, res) in _lib.SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    rd = lib.crucible_debug_decode_stamps
    rd.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                   ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
    rd.restype = ctypes.c_int
    g = Gpu(0)
    g.lib = lib
    g._workspaces = {}
    return g, rd


def _read(rd, rows=8192, clear=0):
    khz, slots = ctypes.c_int(0), ctypes.c_int(0)
    buf = np.zeros((rows, 10), np.uint64)
    assert rd(buf.ctypes.data, rows, clear, ctypes.byref(khz), ctypes.byref(slots)) == 0
    assert slots.value == 10 and khz.value > 0
    return buf


def test_stamped_twin_matches_product_and_stamps_are_ordered(dev, gpu):
    if not os.path.exists(_build.STAMPS_LIB_PATH):
        pytest.skip("stamped library not built")
    twin, rd = _twin_gpu()
    rd(None, 0, 1, ctypes.byref(ctypes.c_int()), ctypes.byref(ctypes.c_int()))  # clear
    batch, n_head, n_kv, max_seq, n_pages = 16, 12, 3, 2048, 8192
    kv = n_kv * 64
    stride = max_seq // 16
    rng = np.random.default_rng(4242)
    lens = rng.integers(64, max_seq, size=batch).astype(np.int32)
    perm = rng.permutation(n_pages).astype(np.int32)
    tables = np.zeros((batch, stride), np.int32)
    cur = 0
    for b, n in enumerate(lens):
        k = -(-int(n) // 16)
        tables[b, :k] = perm[cur:cur + k]
        cur += k
    g = torch.Generator(device="cpu").manual_seed(7)
    n = pool_elems(n_pages, 1, kv)
    k_pool = torch.randn(n, generator=g).half().to(dev)
    v_pool = torch.randn(n, generator=g).half().to(dev)
    q = torch.randn(batch, n_head * 64, generator=g).half().to(dev)
    k_new = torch.randn(batch, kv, generator=g).to(dev)
    v_new = torch.randn(batch, kv, generator=g).to(dev)
    d_tab = torch.from_numpy(tables).to(dev)
    d_len = torch.from_numpy(lens).to(dev)
    d_pos = torch.from_numpy(lens - 1).to(dev)
    results = []
    for g_run in (gpu, twin):
        kp, vp = k_pool.clone(), v_pool.clone()
        out = torch.full((batch, n_head * 64), -1.0, device=dev)
        for _ in range(2):  # the second launch finds the counters left at zero
            g_run.attention_decode_paged_append(q, k_new, v_new, kp, vp, out, d_tab, d_pos,
                                                d_len, batch, n_head, n_kv, 64, stride, 1, 0,
                                                kv, max_seq)
        torch.cuda.synchronize()
        results.append((out.cpu(), kp.cpu(), vp.cpu()))
    for what, a, b in zip(("out", "k pool", "v pool"), *results):
        bits = torch.int16 if a.dtype == torch.float16 else torch.int32
        assert torch.equal(a.view(bits), b.view(bits)), f"{what} differs from the product's"

    st = _read(rd)
    meta = st[:, 9]
    kind = (meta >> np.uint64(52)) & np.uint64(0xF)
    att = (st[:, 0] != 0) & (kind == 0) & (st[:, 6] != 0)
    t = st[att].astype(np.int64)
    n_active = (t[:, 9] >> 32) & 0xFFFF
    last = ((t[:, 9] >> 48) & 1).astype(bool)
    b_of = t[:, 9] & 0xFFFF
    g_of = (t[:, 9] >> 16) & 0xFF
    # one attending workgroup per (request, kv head, active split)
    pages = -(-lens.astype(np.int64) // 16)
    splits = -(-pages // 16)  # 16-page splits of the config-3 shape
    assert att.sum() == n_kv * int(splits.sum())
    assert np.all(b_of < batch) and np.all(g_of < n_kv)
    assert np.all(np.diff(t[:, :7], axis=1) >= 0), "phases 0..6 out of order"
    multi = n_active > 1
    assert np.all(t[multi, 7] >= t[multi, 6])
    comb = multi & last
    assert comb.sum() == n_kv * int((splits > 1).sum())  # one combining split per unit
    assert np.all(t[comb, 8] >= t[comb, 7])


def _read_prefill(twin_lib, rows=8192, clear=0):
    rd = twin_lib.crucible_debug_prefill_stamps
    rd.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                   ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
    rd.restype = ctypes.c_int
    khz, slots = ctypes.c_int(0), ctypes.c_int(0)
    buf = np.zeros((rows, 8), np.uint64)
    if clear:
        assert rd(None, 0, 1, ctypes.byref(khz), ctypes.byref(slots)) == 0
    else:
        assert rd(buf.ctypes.data, rows, 0, ctypes.byref(khz), ctypes.byref(slots)) == 0
        assert slots.value == 8 and khz.value > 0
    return buf


@pytest.mark.parametrize("direct", [1, 0], ids=["direct", "lds"])
def test_stamped_twin_prefill_matches_product(dev, gpu, tune, direct):
    """The register-direct (config-1 shape) and LDS-tiled (config-4 shape) prefill kernels of
    the stamped twin give the product's bits, and their stamps run forward: entry <= rows <=
    first key tile <= loop end <= merge (and the write for the direct form)."""
    if not os.path.exists(_build.STAMPS_LIB_PATH):
        pytest.skip("stamped library not built")
    from crucible_amd import workloads as W
    import bench

    tune(prefill_direct=direct)
    twin, _ = _twin_gpu()
    cfg = W.config1_prefill(n_kv_head=12) if direct else W.config4_packed()
    outs = []
    for g_run in (gpu, twin):
        run = bench.prefill_runner(g_run, dev, cfg)[0]
        if g_run is twin:
            _read_prefill(twin.lib, clear=1)
        run()
        torch.cuda.synchronize()
        outs.append(run.out.cpu().clone())
    assert torch.equal(outs[0].view(torch.int32), outs[1].view(torch.int32))
    st = _read_prefill(twin.lib)
    live = (st[:, 0] != 0) & (st[:, 5] != 0)
    assert live.sum() > 0
    t = st[live].astype(np.int64)
    assert np.all(np.diff(t[:, :5], axis=1) >= 0), "entry, rows, first tile, loop, merge out of order"
    if direct:
        assert np.all(t[:, 5] >= t[:, 4])

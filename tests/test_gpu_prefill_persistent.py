"""The persistent 16-row LDS prefill form against the one-workgroup-per-tile grid.

On request (CRUCIBLE_TUNE_PREFILL_PERSIST), a segment prefill whose longest-first grid holds
more row tiles than the chip holds workgroups runs persistent: the grid is the resident
workgroups (or a forced count), each workgroup lists the row tiles that hold rows from the
segment lengths, and serves list positions w, 2G - 1 - w, 2G + w, ... Each tile's arithmetic
is the same code in both forms, so the outputs must be the same bits: over the reference
corpus with grids forced down to 2, 7 and 64 workgroups (many tiles a workgroup, tiles
without rows among the grid's ids), in both precisions of P and both row modes; on config 4
and on a ragged batch (one long prompt packed with short ones, the case the form is for) at
the resident grid and at a forced 3-workgroup grid, over repeated launches; across graph
replays with eager launches between them; and on two streams at once. The ragged batch is
also checked against the f64 oracle under the element gate.
"""
import numpy as np
import pytest
import torch

import attn_cases as A
import test_gpu_prefill as P
from test_gpu_prefill import CASES, Device, run_owners, run_segments

pytestmark = pytest.mark.gpu

_FIXTURES = {}


def _fixture(case):
    if case.name not in _FIXTURES:
        _FIXTURES[case.name] = A.fixture(case)
    return _FIXTURES[case.name]


@pytest.fixture(params=[False, True], ids=["hilo", "p16"])
def lds16(request, tune):
    """The 16-row LDS kernel (the form with the persistent variant), P as hi + lo or P16."""
    tune(prefill_direct=0, prefill_qb=1, prefill_p16=1 if request.param else None)
    saved = P._P16[0]
    P._P16[0] = request.param  # the oracle gate of _packed_config_check follows the form
    yield request.param
    P._P16[0] = saved


def _corpus_outputs(gpu, dev, tune, persist):
    tune(prefill_persist=persist)
    outs = {}
    for case in CASES:
        fx = _fixture(case)
        for runner in (run_segments, run_owners):
            d = Device(fx, dev)
            runner(gpu, d)
            outs[(case.name, runner.__name__)] = d.result().copy()
    return outs


def test_forced_small_grids_match_the_plain_grid_bit_for_bit(gpu, dev, tune, lds16):
    base = _corpus_outputs(gpu, dev, tune, 0)
    for n in (2, 7, 64):
        got = _corpus_outputs(gpu, dev, tune, n)
        for key, want in base.items():
            assert np.array_equal(got[key].view(np.uint32), want.view(np.uint32)), (n, key)


def _ragged():
    from crucible_amd.workloads import prefill_sequences

    # 1 x 600 + 31 x 24 tokens, 16/4 heads: 38 x 32 x 4 = 4,864 longest-first ids, 256 tiles
    return prefill_sequences("ragged-1x600-31x24", [600] + [24] * 31, 16, 4)


def _config4():
    from crucible_amd.workloads import config4_packed

    return config4_packed()


class Packed:
    """A packed prefill on the device (pools filled by the packed append)."""

    def __init__(self, cfg, dev, seed):
        from crucible_amd.paged import segments_from_cu_seqlens

        rng = np.random.default_rng(seed)
        self.cfg = cfg
        rows, kv = cfg.rows, cfg.kv_dim
        owners = np.concatenate([np.full(n, i, np.int32) for i, n in enumerate(cfg.seq_lens)])
        positions = np.concatenate([np.arange(n, dtype=np.int32) for n in cfg.seq_lens])
        n_elem = cfg.n_pages * cfg.n_layer * 16 * kv
        self.stride = cfg.tables.shape[1]
        self.k = torch.zeros(n_elem, dtype=torch.float16, device=dev)
        self.v = torch.zeros(n_elem, dtype=torch.float16, device=dev)
        self.tables = torch.from_numpy(cfg.tables).to(dev)
        self.owners = torch.from_numpy(owners).to(dev)
        self.positions = torch.from_numpy(positions).to(dev)
        self.k_src = torch.from_numpy(rng.standard_normal((rows, kv)).astype(np.float32)).to(dev)
        self.v_src = torch.from_numpy(rng.standard_normal((rows, kv)).astype(np.float32)).to(dev)
        self.q = torch.from_numpy(
            rng.standard_normal((rows, cfg.n_head * 64)).astype(np.float32)).to(dev).half()
        seg, self.max_chunk = segments_from_cu_seqlens(cfg.cu_seqlens)
        self.segments = torch.from_numpy(seg).to(dev)
        self.out = torch.zeros(rows, cfg.n_head * 64, device=dev)

    def append(self, gpu):
        c = self.cfg
        for src, pool, kind in ((self.k_src, self.k, "k"), (self.v_src, self.v, "v")):
            gpu.cache_store_packed_paged(src, pool, self.tables, self.owners, self.positions,
                                         c.rows, c.kv_dim, self.stride, c.n_layer, 0, kind=kind)

    def prefill(self, gpu, out=None):
        c = self.cfg
        gpu.attention_prefill_tiled(self.q, self.k, self.v, None, None,
                                    self.out if out is None else out, self.tables, self.segments,
                                    len(c.seq_lens), self.max_chunk, self.stride, c.n_head,
                                    c.n_kv_head, 64, c.n_layer, 0, c.kv_dim)


def _bits(t):
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint32).copy()


@pytest.mark.parametrize("make", [_config4, _ragged], ids=["config4", "ragged"])
def test_persistent_equals_plain_grid(gpu, dev, tune, lds16, make):
    w = Packed(make(), dev, 41)
    w.append(gpu)
    tune(prefill_persist=0)
    w.prefill(gpu)
    want = _bits(w.out)
    for persist in (1, 3):  # the resident grid, and a forced 3-workgroup grid
        tune(prefill_persist=persist)
        for _ in range(3):
            w.out.fill_(float("nan"))
            w.prefill(gpu)
            assert np.array_equal(_bits(w.out), want), persist


def test_ragged_batch_matches_oracle(gpu, dev, tune, lds16):
    tune(prefill_persist=1)
    P._packed_config_check(gpu, dev, _ragged(), 13)


def test_graph_replays_with_eager_launches_between_them(gpu, dev, tune, lds16):
    tune(prefill_persist=1)
    w = Packed(_ragged(), dev, 42)
    w.append(gpu)
    w.prefill(gpu)
    want = _bits(w.out)
    out_g = torch.zeros_like(w.out)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        w.prefill(gpu, out_g)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            w.prefill(gpu, out_g)
    torch.cuda.synchronize()
    for r in range(4):
        out_g.fill_(float("nan"))
        graph.replay()
        w.out.fill_(float("nan"))
        w.prefill(gpu)  # eager, queued behind the replay
        assert np.array_equal(_bits(out_g), want), f"replay {r}"
        assert np.array_equal(_bits(w.out), want), f"eager after replay {r}"


def test_two_streams_at_once(gpu, dev, tune, lds16):
    tune(prefill_persist=1)
    a, b = Packed(_ragged(), dev, 43), Packed(_config4(), dev, 44)
    for w in (a, b):
        w.append(gpu)
        w.prefill(gpu)
    want_a, want_b = _bits(a.out), _bits(b.out)
    s1, s2 = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    for s in (s1, s2):
        s.wait_stream(torch.cuda.current_stream(dev))
    outs_a = [torch.full_like(a.out, float("nan")) for _ in range(6)]
    outs_b = [torch.full_like(b.out, float("nan")) for _ in range(6)]
    torch.cuda.synchronize()
    for oa, ob in zip(outs_a, outs_b):  # interleaved, no synchronisation between the streams
        with torch.cuda.stream(s1):
            a.prefill(gpu, oa)
        with torch.cuda.stream(s2):
            b.prefill(gpu, ob)
    torch.cuda.synchronize()
    for i, (oa, ob) in enumerate(zip(outs_a, outs_b)):
        assert np.array_equal(_bits(oa), want_a), f"stream 1 launch {i}"
        assert np.array_equal(_bits(ob), want_b), f"stream 2 launch {i}"

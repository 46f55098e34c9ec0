"""Causal and packed prefill parity.

The reference's attention corpus (gpu_attention_validation.rs:431-509: page boundaries,
offsets, singles up to 1024, packed 16x16..2x512, ragged rows at four Q-scale profiles) runs
through every prefill entry point (segments, owners/positions, params, contiguous) and is
compared with the f64 oracle on every element under the reference's element gate
(|d| <= 2e-5 + 2e-5 |ref|, :20-22) and the north-star max-abs 2e-3. Structural contracts are
exact: future-page poison leaves outputs bit-identical (:597-632), descriptor composition,
order and page reuse leave each request's bits unchanged (:639-682), and output rows outside
the written range keep their sentinel (:23, :271-287). Both prefill kernels (LDS-tiled and
register-direct) run every test in both precisions of P: the default fp16 hi + lo pair
(about 22 bits, the reference's gate as it stands) and the opt-in single fp16 operand (P16,
gated with the rounding term 2^-11 sum w|v| added to the element gate); the LDS-tiled form runs
with 16 rows per wave and with 32 (the 32x32-MFMA kernel, and once over the corpus the
16x16 kernel of that shape).
"""
import numpy as np
import pytest
import torch

import attn_cases as A
import oracle
from gates import element_gate

pytestmark = pytest.mark.gpu


_P16 = [False]  # precision of the running test's prefill_form


@pytest.fixture(autouse=True, params=["lds", "lds32", "direct", "lds-p16", "lds32-p16",
                                        "direct-p16"])
def prefill_form(request, tune):
    """Every test runs through every prefill kernel: the LDS-tiled form with 16 rows per wave
    and with 32 (the 32x32-MFMA kernel), and the register-direct form (the library picks one
    by grid size; the overrides force it), each with P as fp16 hi + lo (the default, under
    the reference's unwidened gate) and as one fp16 operand (P16)."""
    form = request.param
    _P16[0] = form.endswith("-p16")
    tune(prefill_direct=1 if form.startswith("direct") else 0,
         prefill_p16=1 if _P16[0] else None,
         prefill_qb=2 if form.startswith("lds32") else 1 if form.startswith("lds") else None)
    return form


_ORACLE = {}


def corpus_oracle(case):
    """(fixture, f64 oracle output, oracle over |V|) of a corpus case, computed once per
    session and shared by the six prefill forms."""
    if case.name not in _ORACLE:
        fx = A.fixture(case)
        _ORACLE[case.name] = (fx, A.oracle_out(fx), A.oracle_abs_v(fx))
    return _ORACLE[case.name]


def gate(got, want, what, fx=None, q=None, vabs=None, out_f16=False):
    """element_gate with the P16 rounding term when the running form carries P16 (vabs from
    the oracle over |V| of fx, or given)."""
    if _P16[0] and vabs is None:
        vabs = A.oracle_abs_v(fx, q=q)
    return element_gate(got, want, what, out_f16=out_f16, vabs=vabs if _P16[0] else None)


def _dev(a, dev):
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.float16).copy()).to(dev)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


class Device:
    def __init__(self, fx, dev, q_dtype=torch.float32):
        self.fx = fx
        self.q = torch.from_numpy(fx.q).to(dev).to(q_dtype)
        self.k = _dev(fx.k_pool, dev)
        self.v = _dev(fx.v_pool, dev)
        self.tables = _dev(fx.tables, dev)
        self.owners = _dev(fx.owners, dev)
        self.positions = _dev(fx.positions, dev)
        self.segments = _dev(fx.segments, dev)
        self.out = torch.full((fx.rows * A.D + 64,), A.SENTINEL, dtype=torch.float32, device=dev)

    def reset(self):
        self.out.fill_(A.SENTINEL)

    def result(self):
        torch.cuda.synchronize()
        host = self.out.cpu().numpy()
        assert np.all(host[self.fx.rows * A.D:] == A.SENTINEL), "output guard overwritten"
        body = host[:self.fx.rows * A.D].reshape(self.fx.rows, A.D)
        assert np.all(np.isfinite(body)), "nonfinite output"
        return body


def run_segments(gpu, d):
    fx = d.fx
    gpu.attention_prefill_tiled(d.q, d.k, d.v, None, None, d.out, d.tables, d.segments,
                                len(fx.case.slices), fx.max_chunk, A.STRIDE, A.HEADS, A.KV_HEADS,
                                A.HD, A.LAYERS, A.LAYER, A.KD, False, 1024)


def run_owners(gpu, d):
    fx = d.fx
    gpu.attention_prefill_packed(d.q, d.k, d.v, d.out, d.tables, d.owners, d.positions, fx.rows,
                                 A.STRIDE, A.HEADS, A.KV_HEADS, A.HD, A.LAYERS, A.LAYER, A.KD,
                                 A.CONTEXT)


CASES = A.cases()


@pytest.mark.parametrize("case", CASES, ids=[c.name for c in CASES])
def test_corpus_segments_and_owners_match_oracle(gpu, dev, case):
    fx, want, vabs = corpus_oracle(case)
    vabs = vabs if _P16[0] else None
    d = Device(fx, dev)
    errs = []
    for runner in (run_segments, run_owners):
        d.reset()
        runner(gpu, d)
        errs.append(gate(d.result(), want, f"{case.name} {runner.__name__}", vabs=vabs))
    print(f"{case.name}: segments {errs[0]:.3e} owners {errs[1]:.3e}")


FUZZ = A.fuzz_cases()
_FUZZ_ORACLE = {}


def _fuzz_oracle():
    """f64 oracle outputs of the 64 fuzz cases, and of the same cases over |V| (the P16
    term), computed once per session on up to 16 host threads (the C oracle releases the
    interpreter lock)."""
    if not _FUZZ_ORACLE:
        import concurrent.futures
        import os

        workers = max(1, min(16, len(os.sched_getaffinity(0))))
        with concurrent.futures.ThreadPoolExecutor(workers) as ex:
            outs = list(ex.map(lambda c: A.oracle_out(A.fixture(c)), FUZZ))
            absv = list(ex.map(lambda c: A.oracle_abs_v(A.fixture(c)), FUZZ))
        _FUZZ_ORACLE.update({c.name: (o, a) for c, o, a in zip(FUZZ, outs, absv)})
    return _FUZZ_ORACLE


@pytest.mark.timeout(300)
def test_fuzz_corpus_matches_oracle(gpu, dev):
    """The reference's 64 fuzz cases (seed 20260908: 1..16 requests of up to 257 rows at
    random starts, the four Q profiles) through the segment and owners forms; every element
    against the f64 oracle. The reference checks its fuzz cases only against its own
    reference kernel; here the oracle covers every element."""
    want_all = _fuzz_oracle()
    worst = 0.0
    for case in FUZZ:
        fx = A.fixture(case)
        d = Device(fx, dev)
        for runner in (run_segments, run_owners):
            d.reset()
            runner(gpu, d)
            want, vabs = want_all[case.name]
            worst = max(worst, gate(d.result(), want, f"{case.name} {runner.__name__}",
                                    vabs=vabs))
    print(f"fuzz corpus ({len(FUZZ)} cases): max-abs {worst:.3e}")


@pytest.mark.parametrize("case", [c for c in CASES if c.name.startswith("boundary-")],
                         ids=lambda c: c.name)
def test_future_pages_do_not_affect_output(gpu, dev, case):
    fx = A.fixture(case)
    if case.slices[0].start + case.slices[0].len >= A.CONTEXT:
        pytest.skip("no future page inside the context")
    poisoned = A.fixture(case, poison_future=True)
    for runner in (run_segments, run_owners):
        d = Device(fx, dev)
        runner(gpu, d)
        clean = d.result()
        p = Device(poisoned, dev)
        runner(gpu, p)
        assert np.array_equal(clean.view(np.uint32), p.result().view(np.uint32))


def test_repeated_launches_are_bit_identical(gpu, dev):
    """The same call twice gives the same bits: every reduction has a fixed order, and no
    tile is read before it has landed or after it is reused."""
    for case in [c for c in CASES if c.name in ("single-1024", "offset-255", "4x256", "ragged-profile-1")]:
        fx = A.fixture(case)
        d = Device(fx, dev)
        run_segments(gpu, d)
        first = d.result().copy()
        for _ in range(3):
            d.reset()
            run_segments(gpu, d)
            assert np.array_equal(d.result().view(np.uint32), first.view(np.uint32)), case.name


def test_grid_orders_are_bit_identical(gpu, dev, tune):
    """The longest-first grid (the last row tiles of every request dispatched first, the
    default) and the plain (x, row tile, request) grid only place the workgroups: the
    outputs are the same bits."""
    for case in [c for c in CASES if c.name in ("4x256", "ragged-profile-2", "offset-255")]:
        fx = A.fixture(case)
        outs = []
        for order in ("1", "0"):
            tune(prefill_heavy_first=order)
            for runner in (run_segments, run_owners):
                d = Device(fx, dev)
                runner(gpu, d)
                outs.append(d.result().copy())
        assert np.array_equal(outs[0].view(np.uint32), outs[2].view(np.uint32)), case.name
        assert np.array_equal(outs[1].view(np.uint32), outs[3].view(np.uint32)), case.name


def test_single_sequence_params_and_contiguous_forms(gpu, dev):
    """attention_prefill_paged (params[5] offset) and attention_prefill (contiguous)."""
    for case in [c for c in CASES if c.name in ("single-1024", "single-941", "offset-255")]:
        fx, want, vabs_all = corpus_oracle(case)
        d = Device(fx, dev)
        s0 = case.slices[0]
        rows = s0.len
        params = _dev(np.array([0, 0, 0, 0, 0, s0.start], np.int32), dev)
        gpu.attention_prefill_paged(d.q[:rows], d.k, d.v, d.out, d.tables[0], rows,
                                    A.HEADS, A.KV_HEADS, A.HD, A.LAYERS, A.LAYER, A.KD,
                                    A.CONTEXT, params)
        got = d.result()[:rows]
        gate(got, want[:rows], f"{case.name} params form",
             vabs=vabs_all[:rows] if _P16[0] else None)
        # contiguous cache holding the same history for that request at layer 1
        cap = A.CONTEXT
        k_c = np.zeros(A.LAYERS * cap * A.KD, np.uint16)
        v_c = np.zeros_like(k_c)
        n_hist = s0.start + s0.len
        kd = oracle.f32_to_f16_bits(oracle.gather(0, fx.k_pool, fx.tables[0], n_hist, A.KD,
                                                  A.LAYERS, A.LAYER))
        vd = oracle.f32_to_f16_bits(oracle.gather(1, fx.v_pool, fx.tables[0], n_hist, A.KD,
                                                  A.LAYERS, A.LAYER))
        for kind, cache, src in ((0, k_c, kd), (1, v_c, vd)):
            oracle.cache_store(oracle.STORE_CONTIG, kind, cache, src, rows=n_hist, kv_dim=A.KD,
                               layer_base=A.LAYER * cap * A.KD, pos_offset=0)
        d.reset()
        gpu.attention_prefill(d.q[:rows], _dev(k_c, dev), _dev(v_c, dev), d.out, rows,
                              A.HEADS, A.KV_HEADS, A.HD, cap, A.KD, A.LAYER * cap * A.KD,
                              s0.start)
        got_c = d.result()[:rows]
        # same keys, same arithmetic: the contiguous form is bit-identical to the paged one
        assert np.array_equal(got_c.view(np.uint32), got.view(np.uint32))


GPU_PAGED_LENS = [1, 7, 15, 16, 17, 31, 32, 33, 64, 127, 128, 129, 256, 511, 512, 1023]


def _contiguous_caches(fx, n_hist, dev):
    """A contiguous cache ([layer][cap][kv_dim], layer 1) holding request 0's first n_hist
    rows, gathered from the fixture's pools: the same fp16 bits the paged forms read."""
    cap = A.CONTEXT
    k_c = np.zeros(A.LAYERS * cap * A.KD, np.uint16)
    v_c = np.zeros_like(k_c)
    kd = oracle.f32_to_f16_bits(oracle.gather(0, fx.k_pool, fx.tables[0], n_hist, A.KD,
                                              A.LAYERS, A.LAYER))
    vd = oracle.f32_to_f16_bits(oracle.gather(1, fx.v_pool, fx.tables[0], n_hist, A.KD,
                                              A.LAYERS, A.LAYER))
    for kind, cache, src in ((0, k_c, kd), (1, v_c, vd)):
        oracle.cache_store(oracle.STORE_CONTIG, kind, cache, src, rows=n_hist, kv_dim=A.KD,
                           layer_base=A.LAYER * cap * A.KD, pos_offset=0)
    return _dev(k_c, dev), _dev(v_c, dev)


def test_paged_equals_contiguous_over_the_gpu_paged_lengths(gpu, dev):
    """The reference's gpu-paged check (main.rs:106-111, 1253-1257): for every length of its
    list, a prompt of that many rows (positions 0..L-1) through the params form and the
    segment form on the paged pool, and through the contiguous form on a cache holding the
    same rows. Paged must equal contiguous bit for bit, in both paged forms; every output
    is also checked against the f64 oracle."""
    for L in GPU_PAGED_LENS:
        case = A.Case(f"gpu-paged-{L}", [A.Slice(0, 0, L)], A.SEED + L, 0)
        if case.name not in _ORACLE:
            fx = A.fixture(case)
            _ORACLE[case.name] = (fx, A.oracle_out(fx), A.oracle_abs_v(fx))
        fx, want, vabs = _ORACLE[case.name]
        d = Device(fx, dev)
        params = _dev(np.zeros(6, np.int32), dev)
        gpu.attention_prefill_paged(d.q[:L], d.k, d.v, d.out, d.tables[0], L, A.HEADS,
                                    A.KV_HEADS, A.HD, A.LAYERS, A.LAYER, A.KD, A.CONTEXT, params)
        got_p = d.result()[:L].copy()
        d.reset()
        run_segments(gpu, d)
        got_s = d.result()[:L].copy()
        k_c, v_c = _contiguous_caches(fx, L, dev)
        d.reset()
        gpu.attention_prefill(d.q[:L], k_c, v_c, d.out, L, A.HEADS, A.KV_HEADS, A.HD,
                              A.CONTEXT, A.KD, A.LAYER * A.CONTEXT * A.KD, 0)
        got_c = d.result()[:L].copy()
        assert np.array_equal(got_p.view(np.uint32), got_c.view(np.uint32)), f"params, L={L}"
        assert np.array_equal(got_s.view(np.uint32), got_c.view(np.uint32)), f"segments, L={L}"
        gate(got_c, want[:L], f"gpu-paged L={L}", vabs=vabs[:L] if _P16[0] else None)


def test_composition_order_and_page_reuse_invariance(gpu, dev):
    """gpu_attention_validation.rs:639-682: each request's bits are independent of which other
    requests share the call, their order, and the physical pages assigned."""
    expected = {}
    checks = 0
    for count in (16, 1, 8, 2, 4, 16):
        for order in range(3):
            case = A.homogeneous("composition", count, 17, 511, A.SEED + count + order)
            if order == 1:
                case.slices.reverse()
            if order == 2:
                k = count // 2
                case.slices = case.slices[k:] + case.slices[:k]
            fx = A.fixture(case)
            for runner in (run_segments, run_owners):
                d = Device(fx, dev)
                runner(gpu, d)
                out = d.result()
                for row, s in enumerate(case.slices):
                    bits = out[row * 17:(row + 1) * 17].view(np.uint32).tobytes()
                    key = (runner.__name__, s.id)
                    if key in expected:
                        assert bits == expected[key], f"{runner.__name__} request {s.id}"
                        checks += 1
                    else:
                        expected[key] = bits
    assert checks > 50


def test_fp16_query_and_fp16_output(gpu, dev):
    case = [c for c in CASES if c.name == "ragged-profile-0"][0]
    fx = A.fixture(case)
    q16 = fx.q.astype(np.float16).astype(np.float32)
    want = A.oracle_out(fx, q=q16)
    d = Device(fx, dev, q_dtype=torch.float16)
    out16 = torch.zeros(fx.rows, A.D, dtype=torch.float16, device=dev)
    gpu.attention_prefill_tiled(d.q, d.k, d.v, None, None, out16, d.tables, d.segments,
                                len(case.slices), fx.max_chunk, A.STRIDE, A.HEADS, A.KV_HEADS,
                                A.HD, A.LAYERS, A.LAYER, A.KD)
    torch.cuda.synchronize()
    gate(out16.float().cpu().numpy(), want, "fp16 query and output", fx=fx, q=q16, out_f16=True)


def _packed_config_check(gpu, dev, cfg, seed):
    """Append every sequence's K/V through the packed scatter, then segment prefill."""
    rng = np.random.default_rng(seed)
    kv = cfg.kv_dim
    rows = cfg.rows
    owners = np.concatenate([np.full(n, i, np.int32) for i, n in enumerate(cfg.seq_lens)])
    positions = np.concatenate([np.arange(n, dtype=np.int32) for n in cfg.seq_lens])
    k_src = oracle.f32_to_f16_bits(rng.standard_normal((rows, kv)))
    v_src = oracle.f32_to_f16_bits(rng.standard_normal((rows, kv)))
    q = oracle.f32_to_f16_bits(rng.standard_normal((rows, cfg.n_head * 64)))
    n_elem = cfg.n_pages * cfg.n_layer * 16 * kv
    stride = cfg.tables.shape[1]
    k_pool = torch.zeros(n_elem, dtype=torch.float16, device=dev)
    v_pool = torch.zeros(n_elem, dtype=torch.float16, device=dev)
    d_tab, d_own, d_pos = _dev(cfg.tables, dev), _dev(owners, dev), _dev(positions, dev)
    gpu.cache_store_packed_paged(_dev(k_src, dev), k_pool, d_tab, d_own, d_pos, rows, kv, stride,
                                 cfg.n_layer, 0, kind="k")
    gpu.cache_store_packed_paged(_dev(v_src, dev), v_pool, d_tab, d_own, d_pos, rows, kv, stride,
                                 cfg.n_layer, 0, kind="v")
    from crucible_amd.paged import segments_from_cu_seqlens
    seg, max_chunk = segments_from_cu_seqlens(cfg.cu_seqlens)
    out = torch.zeros(rows, cfg.n_head * 64, device=dev)
    gpu.attention_prefill_tiled(_dev(q, dev), k_pool, v_pool, None, None, out, d_tab,
                                _dev(seg, dev), len(cfg.seq_lens), max_chunk, stride, cfg.n_head,
                                cfg.n_kv_head, 64, cfg.n_layer, 0, kv)
    torch.cuda.synchronize()
    kp = k_pool.cpu().numpy().view(np.uint16)
    vp = v_pool.cpu().numpy().view(np.uint16)
    key = ("config", cfg.name, cfg.n_kv_head, seed)
    if key not in _ORACLE:  # the same seeded pools in every form: one oracle run per session
        args = dict(table_index=owners, n_head=cfg.n_head, n_kv_head=cfg.n_kv_head, head_dim=64,
                    table_stride=stride, n_layer=cfg.n_layer, layer=0)
        qf = oracle.f16_bits_to_f32(q)
        _ORACLE[key] = (
            kp.copy(), vp.copy(),
            oracle.attention_paged_rows(qf, kp, vp, cfg.tables, positions + 1, **args),
            oracle.attention_paged_rows(qf, kp, vp & np.uint16(0x7FFF), cfg.tables,
                                        positions + 1, **args))
    kp0, vp0, want, vabs = _ORACLE[key]
    # the pools this form's appends wrote are the bytes the oracle ran on
    assert np.array_equal(kp, kp0) and np.array_equal(vp, vp0)
    err = gate(out.cpu().numpy(), want, cfg.name, vabs=vabs if _P16[0] else None)
    print(f"{cfg.name}: max-abs {err:.3e}")


def test_qb2_on_16x16_mfma_matches_oracle(gpu, dev, tune, prefill_form):
    """32 rows per wave on 16x16 MFMAs (CRUCIBLE_TUNE_PREFILL_M32 = 0, the other kernel for
    that shape) over the corpus, both row modes, in the running form's precision."""
    if not prefill_form.startswith("lds32"):
        pytest.skip("the 32-row shape only")
    tune(prefill_m32=0)
    for case in CASES:
        fx, want, vabs = corpus_oracle(case)
        vabs = vabs if _P16[0] else None
        d = Device(fx, dev)
        for runner in (run_segments, run_owners):
            d.reset()
            runner(gpu, d)
            gate(d.result(), want, f"{case.name} {runner.__name__} (16x16, 32 rows)", vabs=vabs)


def test_config1_causal_prefill_512(gpu, dev):
    from crucible_amd.workloads import config1_prefill
    for n_kv in (12, 3):
        _packed_config_check(gpu, dev, config1_prefill(n_kv_head=n_kv), 11)


def test_config4_packed_varlen_350m(gpu, dev):
    from crucible_amd.workloads import config4_packed
    _packed_config_check(gpu, dev, config4_packed(), 12)

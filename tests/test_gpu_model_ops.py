"""Decode-step glue kernels against numpy float64 restatements of the reference CPU ops.

The reference arithmetic (engine/src/ops.rs): matvec (:17-32) rounds an f64 sum of f64
products to f32 once; rmsnorm (:39-52) takes the f64 mean of squares, scale =
1/sqrt(mean + eps) in f64, h = f32(f64(x) * scale) * w; silu (:83-85) is
g / (1 + exp(-g)); RoPE (:124-135) pairs element i with i + 32. numpy's float64 GEMM sums
in another order than the f64 MFMA, so a result may differ from it only where the two f64
sums straddle an f32 rounding boundary: the bar is bit-identity on all but a handful of
elements and 1 ulp on those. RoPE and the split are exact. Results must also be
bit-identical from run to run (fixed reduction order, no atomics).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

EPS = np.float32(1e-6)


def _ulps(a, b):
    ai = a.astype(np.float32).view(np.int32).astype(np.int64)
    bi = b.astype(np.float32).view(np.int32).astype(np.int64)
    return np.abs(ai - bi)


def _assert_f64_contract(got, want, what):
    d = _ulps(got, want)
    n_off = int((d > 0).sum())
    assert d.max() <= 1, f"{what}: {d.max()} ulps"
    assert n_off <= max(2, got.size // 20000), f"{what}: {n_off} of {got.size} off by 1 ulp"


def _rms_ref(x, w):
    x64 = x.astype(np.float64)
    scale = 1.0 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + np.float64(EPS))
    return (x64 * scale).astype(np.float32) * w


def _mat(rng, shape, std):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float16)


# linear_tile tuning: the launcher's choice, or forced: 4 or 16 columns (the decode
# tilings), 32 (the output-tiled products of prompt-sized batches; k_in % 64 == 0 only)
TILES = ["auto", "4", "16", "32"]


@pytest.mark.parametrize("rows,n_out,k_in", [(1, 1152, 768), (16, 768, 768), (5, 200, 2048),
                                             (33, 768, 256), (16, 50257, 768), (4, 256, 704),
                                             (2, 64, 96), (33, 16400, 256), (3, 16400, 1056),
                                             (7, 203, 160)])
@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("tile", TILES)
def test_linear_matches_f64_matvec(gpu, dev, tune, rows, n_out, k_in, norm, tile):
    if tile != "auto":
        if n_out >= 16 * 1024 and tile != "32":
            pytest.skip("the vocabulary-sized outputs take the persistent wide kernel")
        tune(linear_tile=tile)
    rng = np.random.default_rng(rows * 7 + n_out + k_in + norm)
    x = rng.standard_normal((rows, k_in), dtype=np.float32)
    w = _mat(rng, (n_out, k_in), 0.02)
    nw = (1.0 + 0.1 * rng.standard_normal(k_in)).astype(np.float32)
    h = _rms_ref(x, nw) if norm else x
    want = (h.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32)
    dx, dw = torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev)
    dn = torch.from_numpy(nw).to(dev) if norm else None
    out = torch.full((rows, n_out), np.nan, dtype=torch.float32, device=dev)
    gpu.linear_f64acc(dx, dw, out, norm_w=dn, eps=float(EPS))
    got = out.cpu().numpy()
    _assert_f64_contract(got, want, "linear")
    again = torch.empty_like(out)
    gpu.linear_f64acc(dx, dw, again, norm_w=dn, eps=float(EPS))
    assert torch.equal(out, again), "not deterministic"


@pytest.mark.parametrize("tile", TILES)
def test_linear_residual_in_place(gpu, dev, tune, tile):
    if tile != "auto":
        tune(linear_tile=tile)
    rng = np.random.default_rng(5)
    rows, n_out, k_in = 16, 768, 2048
    a = rng.standard_normal((rows, k_in), dtype=np.float32)
    w = _mat(rng, (n_out, k_in), 0.02)
    x = rng.standard_normal((rows, n_out), dtype=np.float32)
    y = (a.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32)
    want = x + y
    dx = torch.from_numpy(x).to(dev)
    gpu.linear_f64acc(torch.from_numpy(a).to(dev), torch.from_numpy(w).to(dev), dx, resid=dx)
    got = dx.cpu().numpy()
    # the residual add is exact f32 once y is; compare through y's contract
    _assert_f64_contract(got - x, want - x, "residual")
    assert np.abs(got - want).max() <= 4 * np.abs(want).max() * 2.0 ** -24


@pytest.mark.parametrize("rows,hidden,k_in", [(16, 2048, 768), (5, 2045, 96), (21, 130, 1056),
                                             (37, 1000, 704)])
@pytest.mark.parametrize("tile", TILES)
def test_swiglu_matches_reference_ops(gpu, dev, tune, rows, hidden, k_in, tile):
    if tile != "auto":
        tune(linear_tile=tile)
    rng = np.random.default_rng(9 + hidden)
    x = rng.standard_normal((rows, k_in), dtype=np.float32)
    wg = _mat(rng, (hidden, k_in), 0.05)
    wu = _mat(rng, (hidden, k_in), 0.05)
    nw = np.ones(k_in, np.float32)
    h = _rms_ref(x, nw).astype(np.float64)
    g = (h @ wg.astype(np.float64).T).astype(np.float32)
    u = (h @ wu.astype(np.float64).T).astype(np.float32)
    want = (g / (np.float32(1.0) + np.exp(-g))) * u
    out = torch.empty((rows, hidden), dtype=torch.float32, device=dev)
    gpu.linear_swiglu_f64acc(torch.from_numpy(x).to(dev), torch.from_numpy(wg).to(dev),
                             torch.from_numpy(wu).to(dev), out,
                             norm_w=torch.from_numpy(nw).to(dev), eps=float(EPS))
    got = out.cpu().numpy()
    # exp may differ by an ulp between libraries: a few ulps of the product at most
    assert np.all(np.abs(got - want) <= 8 * 2.0 ** -24 * np.abs(want) + 1e-30)


# the decode step's four projections at batch 16, and ragged shapes
PREFETCH_SHAPES = [("qkv", 16, 1280, 768, True, False), ("o", 16, 768, 768, False, True),
                   ("down", 16, 768, 2048, False, True), ("ragged", 5, 200, 2048, True, False),
                   ("small", 7, 203, 160, False, True)]


@pytest.mark.parametrize("tile", ["auto", "4", "16"])
@pytest.mark.parametrize("pf_bytes", [100, 2 << 20, 64 << 20])
def test_prefetch_variants_write_the_plain_products(gpu, dev, tune, tile, pf_bytes):
    """The _prefetch entry points, with a region of one line, of a projection's weights and
    of more than the grid fetches (128 KB a workgroup), write the plain entry points' bits;
    the region is read only. The tuning key's off setting does the same."""
    if tile != "auto":
        tune(linear_tile=tile)
    rng = np.random.default_rng(pf_bytes % 1000 + len(tile))
    region = torch.from_numpy(rng.integers(0, 255, pf_bytes, dtype=np.uint8)).to(dev)
    region_before = region.clone()
    for name, rows, n_out, k_in, norm, resid in PREFETCH_SHAPES:
        x = torch.from_numpy(rng.standard_normal((rows, k_in), dtype=np.float32)).to(dev)
        w = torch.from_numpy(_mat(rng, (n_out, k_in), 0.02)).to(dev)
        nw = torch.from_numpy((1.0 + 0.1 * rng.standard_normal(k_in)).astype(np.float32)).to(dev)
        r = torch.from_numpy(rng.standard_normal((rows, n_out), dtype=np.float32)).to(dev)
        kw = dict(norm_w=nw if norm else None, eps=float(EPS))
        want = r.clone()
        gpu.linear_f64acc(x, w, want, resid=want if resid else None, **kw)
        for setting in (None, 0):
            tune(linear_prefetch=setting)
            got = r.clone()
            gpu.linear_f64acc(x, w, got, resid=got if resid else None, prefetch=region, **kw)
            assert torch.equal(got, want), (name, setting)
        tune(linear_prefetch=None)
        wg = torch.from_numpy(_mat(rng, (n_out, k_in), 0.05)).to(dev)
        want = torch.full((rows, n_out), np.nan, device=dev)
        gpu.linear_swiglu_f64acc(x, w, wg, want, **kw)
        got = torch.full_like(want, np.nan)
        gpu.linear_swiglu_f64acc(x, w, wg, got, prefetch=region, **kw)
        assert torch.equal(got, want), (name, "swiglu")
    assert torch.equal(region, region_before)


def test_rmsnorm_rows(gpu, dev):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((7, 768), dtype=np.float32) * 3).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(768)).astype(np.float32)
    out = torch.empty((7, 768), dtype=torch.float32, device=dev)
    gpu.rmsnorm_rows(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev), out, float(EPS))
    _assert_f64_contract(out.cpu().numpy(), _rms_ref(x, w), "rmsnorm")


def test_rope_split_is_exact(gpu, dev):
    from crucible_amd.gpu_model import rope_tables

    rng = np.random.default_rng(4)
    rows, nh, nkv, cap = 16, 12, 3, 1024
    cos, sin = rope_tables(64, cap, 10000.0)
    qkv = rng.standard_normal((rows, (nh + 2 * nkv) * 64), dtype=np.float32)
    pos = rng.integers(0, cap, rows).astype(np.int32)
    q = torch.empty((rows, nh * 64), dtype=torch.float32, device=dev)
    k = torch.empty((rows, nkv * 64), dtype=torch.float32, device=dev)
    v = torch.empty((rows, nkv * 64), dtype=torch.float32, device=dev)
    gpu.rope_split_qkv(torch.from_numpy(qkv).to(dev), q, k, v, torch.from_numpy(cos).to(dev),
                       torch.from_numpy(sin).to(dev), torch.from_numpy(pos).to(dev), nh, nkv)

    def rot(block, heads):
        out = block.reshape(rows, heads, 64).copy()
        c = cos[pos][:, None, :]
        s = sin[pos][:, None, :]
        lo, hi = out[..., :32].copy(), out[..., 32:].copy()
        out[..., :32] = lo * c - hi * s
        out[..., 32:] = lo * s + hi * c
        return out.reshape(rows, heads * 64)

    d = nh * 64
    assert np.array_equal(q.cpu().numpy(), rot(qkv[:, :d], nh))
    assert np.array_equal(k.cpu().numpy(), rot(qkv[:, d:d + nkv * 64], nkv))
    assert np.array_equal(v.cpu().numpy(), qkv[:, d + nkv * 64:])


@pytest.mark.parametrize("rows", [1003, 2304, 4713])
def test_prefill_sized_projections_keep_the_f64_contract(gpu, dev, rows):
    """The packed prefill runs the same projections over every prompt row at once (config 5:
    about 4,600 rows): q/k/v with the attention norm fused, o and down with the residual add,
    gate/up with SwiGLU, at the 120m preset's shapes, each against numpy float64."""
    rng = np.random.default_rng(rows)
    d, kv, hidden = 768, 192, 2048
    x = rng.standard_normal((rows, d), dtype=np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    wqkv = _mat(rng, (d + 2 * kv, d), 0.02)
    h = _rms_ref(x, nw).astype(np.float64)
    want = (h @ wqkv.astype(np.float64).T).astype(np.float32)
    out = torch.empty((rows, d + 2 * kv), dtype=torch.float32, device=dev)
    dx = torch.from_numpy(x).to(dev)
    gpu.linear_f64acc(dx, torch.from_numpy(wqkv).to(dev), out, norm_w=torch.from_numpy(nw).to(dev),
                      eps=float(EPS))
    _assert_f64_contract(out.cpu().numpy(), want, f"qkv {rows} rows")
    again = torch.empty_like(out)
    gpu.linear_f64acc(dx, torch.from_numpy(wqkv).to(dev), again,
                      norm_w=torch.from_numpy(nw).to(dev), eps=float(EPS))
    assert torch.equal(out, again), "not deterministic"
    # o projection with the residual add in place
    wo = _mat(rng, (d, d), 0.02)
    a = rng.standard_normal((rows, d), dtype=np.float32)
    y = (a.astype(np.float64) @ wo.astype(np.float64).T).astype(np.float32)
    res = dx.clone()
    gpu.linear_f64acc(torch.from_numpy(a).to(dev), torch.from_numpy(wo).to(dev), res, resid=res)
    _assert_f64_contract(res.cpu().numpy() - x, (x + y) - x, f"o + residual {rows} rows")
    # gate/up with SwiGLU, then down
    wg = _mat(rng, (hidden, d), 0.05)
    wu = _mat(rng, (hidden, d), 0.05)
    g = (h @ wg.astype(np.float64).T).astype(np.float32)
    u = (h @ wu.astype(np.float64).T).astype(np.float32)
    want_act = (g / (np.float32(1.0) + np.exp(-g))) * u
    act = torch.empty((rows, hidden), dtype=torch.float32, device=dev)
    gpu.linear_swiglu_f64acc(dx, torch.from_numpy(wg).to(dev), torch.from_numpy(wu).to(dev), act,
                             norm_w=torch.from_numpy(nw).to(dev), eps=float(EPS))
    got_act = act.cpu().numpy()
    assert np.all(np.abs(got_act - want_act) <= 8 * 2.0 ** -24 * np.abs(want_act) + 1e-30)
    wd = _mat(rng, (d, hidden), 0.02)
    want_d = (got_act.astype(np.float64) @ wd.astype(np.float64).T).astype(np.float32)
    down = torch.empty((rows, d), dtype=torch.float32, device=dev)
    gpu.linear_f64acc(act, torch.from_numpy(wd).to(dev), down)
    _assert_f64_contract(down.cpu().numpy(), want_d, f"down {rows} rows")

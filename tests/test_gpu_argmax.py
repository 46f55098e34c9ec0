"""Device greedy selection against the host rule of sampling.rs:141-150 (the oracle's
orc_argmax): the adversarial rows of gpu.rs:2295-2399, NaN at every kind of position,
signed zeros, infinities, and random rows. Index work: the answer must be identical."""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

VOCAB = 50257  # BASELINE config 5 vocabulary (odd, not a multiple of 4)


def _rows(vocab):
    i = np.arange(vocab, dtype=np.float32)
    dense = (np.sin(i * np.float32(0.7391)) * 3.0 - 1.0).astype(np.float32)
    dense[31337 % vocab] = 9.0
    tied = np.full(vocab, -2.0, np.float32)
    tied[[100, 7000 % vocab]] = 5.0
    first = np.full(vocab, -3.0, np.float32)
    first[0] = 1.0
    last = np.full(vocab, -3.0, np.float32)
    last[-1] = 1.0
    close = np.zeros(vocab, np.float32)
    close[4242], close[4243] = np.float32(1.0000001), np.float32(1.0)
    all_neg = (-1.0 - i * np.float32(1e-4)).astype(np.float32)
    nan_first = np.ones(vocab, np.float32)
    nan_first[0] = np.nan
    nan_mid = np.ones(vocab, np.float32)
    nan_mid[500], nan_mid[900] = np.nan, 4.0
    all_nan = np.full(vocab, np.nan, np.float32)
    # NaN as some thread's first element, before the true maximum
    nan_early = np.ones(vocab, np.float32)
    nan_early[[1, 100, 1023]] = np.nan
    nan_early[2000] = 3.0
    # signed zeros: -0.0 first, +0.0 later must not win (equal values)
    zeros = np.full(vocab, -1.0, np.float32)
    zeros[10], zeros[20] = np.float32(-0.0), np.float32(0.0)
    inf = np.zeros(vocab, np.float32)
    inf[[77, 78]] = np.inf
    neg_inf = np.full(vocab, -np.inf, np.float32)
    neg_inf[3000] = -1e30
    only_last_finite = np.full(vocab, np.nan, np.float32)
    only_last_finite[0] = -5.0
    only_last_finite[-1] = 7.0
    return [dense, tied, first, last, close, all_neg, nan_first, nan_mid, all_nan, nan_early,
            zeros, inf, neg_inf, only_last_finite]


@pytest.mark.parametrize("vocab", [VOCAB, 50304, 1, 3, 1025, 4097])
def test_argmax_rows_matches_host_rule(gpu, dev, vocab):
    rows = _rows(vocab) if vocab >= 32000 else []
    rng = np.random.default_rng(vocab)
    for _ in range(16):
        r = rng.standard_normal(vocab).astype(np.float32)
        if vocab > 8 and rng.random() < 0.5:  # a planted tie
            j, k = sorted(rng.choice(vocab, 2, replace=False))
            r[j] = r[k] = np.float32(r.max() + 1.0)
        rows.append(r)
    x = np.stack(rows).astype(np.float32)
    d_x = torch.from_numpy(x).to(dev)
    out = torch.full((x.shape[0],), -7, dtype=torch.int32, device=dev)
    gpu.argmax_rows(d_x, out, x.shape[0], vocab)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = np.array([oracle.argmax(r) for r in x])
    assert np.array_equal(got, want), np.nonzero(got != want)


def test_argmax_batch16_logits(gpu, dev):
    """The config-5 shape: 16 rows of 50257 logits, random with small top-2 gaps."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((16, VOCAB)) * 0.5).astype(np.float32)
    for r in range(16):
        top = int(np.argmax(x[r]))
        x[r, (top + 1 + r * 97) % VOCAB] = np.nextafter(x[r, top], np.float32(-np.inf))
    d_x = torch.from_numpy(x).to(dev)
    out = torch.empty(16, dtype=torch.int32, device=dev)
    gpu.argmax_rows(d_x, out, 16, VOCAB)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), [oracle.argmax(r) for r in x])

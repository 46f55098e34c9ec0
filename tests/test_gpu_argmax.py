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


def test_greedy_advance_matches_host_rule_and_bookkeeping(gpu, dev):
    """The fused greedy tail: tokens by the host rule on the adversarial rows, history
    row `step`, positions and lengths + 1, x = emb[token], step + 1, the counter back at
    0; two calls in a row (the second sees the first's step)."""
    rows_np = _rows(VOCAB)[:14]
    rng = np.random.default_rng(11)
    rows_np += [rng.standard_normal(VOCAB).astype(np.float32) for _ in range(2)]
    n_embd, max_steps = 48, 3
    emb = rng.standard_normal((VOCAB, n_embd)).astype(np.float32)
    d_emb = torch.from_numpy(emb).to(dev)
    rows = len(rows_np)
    tokens = torch.full((rows,), -7, dtype=torch.int32, device=dev)
    history = torch.full((max_steps, rows), -9, dtype=torch.int32, device=dev)
    step = torch.zeros(1, dtype=torch.int64, device=dev)
    positions = torch.arange(rows, dtype=torch.int32, device=dev) * 10
    lens = positions + 1
    done = torch.zeros(1, dtype=torch.int32, device=dev)
    x = torch.full((rows, n_embd), np.nan, dtype=torch.float32, device=dev)
    for call in range(2):
        logits = np.stack(rows_np) if call == 0 else np.stack(rows_np[::-1])
        want = np.array([oracle.argmax(r) for r in logits])
        gpu.greedy_advance(torch.from_numpy(np.ascontiguousarray(logits)).to(dev), d_emb, x,
                           tokens, history, step, positions, lens, done)
        torch.cuda.synchronize()
        assert np.array_equal(tokens.cpu().numpy(), want)
        assert np.array_equal(history[call].cpu().numpy(), want)
        assert np.array_equal(x.cpu().numpy(), emb[want])
        assert int(step.item()) == call + 1
        assert int(done.item()) == 0
        base = np.arange(rows, dtype=np.int32) * 10 + call + 1
        assert np.array_equal(positions.cpu().numpy(), base)
        assert np.array_equal(lens.cpu().numpy(), base + 1)
    assert np.all(history[2].cpu().numpy() == -9)


def test_greedy_advance_past_history_end_skips_the_write(gpu, dev):
    """A step at or past max_steps leaves the history alone (no write out of bounds)."""
    rng = np.random.default_rng(12)
    rows, vocab, n_embd = 4, 1000, 16
    logits = torch.from_numpy(rng.standard_normal((rows, vocab)).astype(np.float32)).to(dev)
    emb = torch.from_numpy(rng.standard_normal((vocab, n_embd)).astype(np.float32)).to(dev)
    history = torch.full((1, rows), -9, dtype=torch.int32, device=dev)
    step = torch.ones(1, dtype=torch.int64, device=dev)
    tokens = torch.empty(rows, dtype=torch.int32, device=dev)
    positions = torch.zeros(rows, dtype=torch.int32, device=dev)
    lens = torch.ones(rows, dtype=torch.int32, device=dev)
    done = torch.zeros(1, dtype=torch.int32, device=dev)
    x = torch.empty((rows, n_embd), dtype=torch.float32, device=dev)
    gpu.greedy_advance(logits, emb, x, tokens, history, step, positions, lens, done)
    torch.cuda.synchronize()
    assert np.all(history.cpu().numpy() == -9)
    assert int(step.item()) == 2
    assert np.array_equal(tokens.cpu().numpy(), logits.cpu().numpy().argmax(axis=1))

"""The beam step's choice on an MI355X through the C ABI (``omni_beam_select``), against torch's own ops on the same
inputs: ``F.log_softmax`` in bf16, the offers of src/omniasr_trt/beam.py:165-170 as torch element-wise ops, and
``topk`` over each group's N x V offers.

* The default path (torch's log-softmax, then the offers and top-k in one launch) makes the choice torch's ops make:
  every group's indices and values are equal bit for bit (ties in value by lower flat index, the order torch.topk
  leaves unspecified).
* The fused path (``fused_log_softmax=True``: the log-softmax in the same launch) sums exp(x - max) in its own order,
  so its logsum can differ from torch's in the last fp32 bit and a logp near a bf16 rounding boundary can round the
  other way (one bf16 step).  Its checks: the chosen indices equal torch's on every group whose best N + 1 offers are
  separated by more than one bf16 step of their logp; every chosen value is within one bf16 step of logp (scaled as
  the offer scales it) of torch's value for the same (row, token), and at least 99.9% are equal bit for bit.
* Exact cases that involve no log-softmax: groups whose rows all ended (only EOS, at each row's score) and identical
  rows (equal offers, taken in flat-index order), on both paths.
"""

import sys

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from omniasr_trt_amd import kernels

pytestmark = pytest.mark.gpu
EOS = 2


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def torch_offers(logits, score, count, ended, n, length_norm):
    """The reference's offers (src/omniasr_trt/beam.py:165-170) as torch ops; also returns logp."""
    logp = F.log_softmax(logits, dim=-1)
    summed = score[:, None] + logp
    if length_norm:
        lead = count.view(-1, n)[:, :1].expand(-1, n).reshape(-1, 1)
        c = count[:, None]
        summed = torch.where(lead > 0, (score[:, None] * c + logp) / (c + 1), summed)
    offers = summed.masked_fill(ended[:, None], float("-inf"))
    offers[:, EOS] = torch.where(ended, score, offers[:, EOS])
    return offers, logp


def choose(offers: np.ndarray, n: int):
    """Each group's n best of its flattened offers: larger value first, then the lower flat index."""
    g = offers.shape[0]
    best = np.empty((g, n), np.float32)
    flat = np.empty((g, n), np.int64)
    for i in range(g):
        row = offers[i]
        order = np.lexsort((np.arange(row.size), -row.astype(np.float64)))[:n]
        best[i], flat[i] = row[order], order
    return best, flat


def inputs(groups, n, vocab, seed, ended_frac=0.2, spread=4.0):
    g = torch.Generator().manual_seed(seed)
    rows = groups * n
    logits = (torch.randn(rows, vocab, generator=g) * spread).to(torch.bfloat16)
    score = (-torch.rand(rows, generator=g) * 30).float()
    count = torch.randint(0, 40, (rows,), generator=g)
    count[::n][: groups // 3] = 0  # some groups whose row 0 has no tokens yet (no length norm for them)
    ended = torch.rand(rows, generator=g) < ended_frac
    return logits, score, count, ended


CASES = [(8, 5, 10288, True), (8, 5, 10288, False), (3, 1, 10288, True), (2, 16, 10288, True), (5, 8, 64, False),
         (4, 4, 16384, True), (1, 5, 8192, True)]


@pytest.mark.parametrize("groups,n,vocab,length_norm", CASES)
def test_beam_select_matches_torch(cuda, groups, n, vocab, length_norm):
    say(f"beam_select groups={groups} beams={n} vocab={vocab} length_norm={length_norm}")
    logits, score, count, ended = inputs(groups, n, vocab, groups * 100 + n * 10 + vocab % 97 + length_norm)
    lg, sc, ct, en = logits.to(cuda), score.to(cuda), count.to(cuda), ended.to(cuda)
    tickets = torch.zeros(groups, dtype=torch.int32, device=cuda)
    best, flat = kernels.beam_select(lg, sc, ct, en, n, length_norm, EOS, tickets=tickets)
    offers, _ = torch_offers(lg, sc, ct, en, n, length_norm)
    want_best, want_flat = choose(offers.view(groups, n * vocab).cpu().numpy(), n)
    np.testing.assert_array_equal(flat.cpu().numpy(), want_flat)
    np.testing.assert_array_equal(best.cpu().numpy(), want_best)
    assert int(tickets.abs().sum()) == 0


@pytest.mark.parametrize("groups,n,vocab,length_norm", CASES)
def test_beam_select_fused_log_softmax(cuda, groups, n, vocab, length_norm):
    say(f"beam_select (fused log-softmax) groups={groups} beams={n} vocab={vocab} length_norm={length_norm}")
    logits, score, count, ended = inputs(groups, n, vocab, groups * 100 + n * 10 + vocab % 97 + length_norm)
    lg, sc, ct, en = logits.to(cuda), score.to(cuda), count.to(cuda), ended.to(cuda)
    best, flat = kernels.beam_select(lg, sc, ct, en, n, length_norm, EOS, fused_log_softmax=True)
    offers, logp = torch_offers(lg, sc, ct, en, n, length_norm)
    off = offers.view(groups, n * vocab).cpu().numpy()
    want_best, want_flat = choose(off, n)
    got_best, got_flat = best.cpu().numpy(), flat.cpu().numpy()
    # One bf16 step of each offer's logp, scaled as the offer scales it (1 / (count + 1) under length norm).
    lp = logp.float().cpu().numpy().reshape(groups, n * vocab)
    cnt = count.numpy().reshape(groups, n)
    lead = cnt[:, :1] > 0
    scale = np.where(length_norm & lead, 1.0 / (cnt + 1), 1.0).repeat(vocab, axis=1)
    step = np.abs(lp) * 2.0 ** -7 * scale + 1e-6
    top_best, top_flat = choose(off, n + 1)
    margin = -np.diff(top_best.astype(np.float64), axis=1)  # gaps between consecutive best offers
    top_step = np.take_along_axis(step, top_flat, axis=1)
    clear = [bool((margin[i] > 2 * top_step[i].max()).all()) for i in range(groups)]
    say(f"  groups with clear margins: {sum(clear)} of {groups}")
    for i in range(groups):
        if clear[i]:
            assert (got_flat[i] == want_flat[i]).all(), (i, got_flat[i], want_flat[i])
    # Values: each chosen (row, token)'s offer within one bf16 step of logp of torch's offer for it.
    tv = np.take_along_axis(off, got_flat, axis=1)
    ts = np.take_along_axis(step, got_flat, axis=1)
    fin = np.isfinite(tv)
    assert (np.isfinite(got_best) == fin).all()
    assert (np.abs(got_best - tv)[fin] <= ts[fin]).all()
    same = float((got_best == tv)[fin].mean()) if fin.any() else 1.0
    say(f"  chosen values equal to torch's offers bit for bit: {same:.4f}")
    assert same >= 0.999
    wfin = np.isfinite(want_best)
    assert (np.abs(got_best - want_best)[wfin] <= np.take_along_axis(step, want_flat, axis=1)[wfin]).all()
    assert int(kernels._select_tickets[torch.cuda.current_device()].abs().sum()) == 0


def test_beam_select_exact_cases(cuda):
    """No log-softmax involved: all-ended groups offer only EOS at each row's score; identical rows tie everywhere."""
    n, vocab = 5, 10288
    g = torch.Generator().manual_seed(77)
    logits = (torch.randn(2 * n, vocab, generator=g) * 3).to(torch.bfloat16)
    logits[n + 3] = logits[n + 1]  # group 1: rows 1 and 3 identical (same logits, score and count)
    score = torch.tensor([-1.5, -0.25, -3.0, -0.25, -2.0, -4.0, -2.5, -7.0, -2.5, -1.0]).float()
    count = torch.full((2 * n,), 7, dtype=torch.long)
    ended = torch.zeros(2 * n, dtype=torch.bool)
    ended[:n] = True  # group 0: every row finished
    for fused in (False, True):
        best, flat = kernels.beam_select(logits.to(cuda), score.to(cuda), count.to(cuda), ended.to(cuda), n, True, EOS,
                                         fused_log_softmax=fused)
        check_exact_cases(logits, score, count, ended, n, vocab, best.cpu(), flat.cpu(), cuda)


def check_exact_cases(logits, score, count, ended, n, vocab, best, flat, cuda):
    # group 0: EOS of each row at its score, best first, equal scores (rows 1 and 3) by row
    assert best[0].tolist() == [-0.25, -0.25, -1.5, -2.0, -3.0]
    assert flat[0].tolist() == [1 * vocab + EOS, 3 * vocab + EOS, 0 * vocab + EOS, 4 * vocab + EOS, 2 * vocab + EOS]
    # group 1: rows 1 and 3 offer the same values, so each of their tokens comes as the pair (row 1, row 3)
    f1 = flat[1].tolist()
    for j, f in enumerate(f1):
        if f // vocab == 3:
            assert (1 * vocab + f % vocab) in f1[:j]
    offers, _ = torch_offers(logits.to(cuda), score.to(cuda), count.to(cuda), ended.to(cuda), n, True)
    tb, tf = offers.view(2, n * vocab).topk(n, dim=-1, sorted=True)
    assert torch.equal(best[0], tb[0].cpu()) and torch.equal(best[1], tb[1].cpu())
    say(f"  ties: torch.topk's indices {tf.tolist()}, ours {flat.tolist()}")


def test_beam_select_refusals(cuda):
    lg = torch.zeros(10, 64, dtype=torch.bfloat16, device=cuda)
    sc = torch.zeros(10, device=cuda)
    ct = torch.zeros(10, dtype=torch.long, device=cuda)
    en = torch.zeros(10, dtype=torch.bool, device=cuda)
    assert not kernels.beam_select_supported(lg.float(), sc, 5)  # fp32 logits
    assert not kernels.beam_select_supported(lg[:, :60], sc, 5)  # V not a multiple of 8
    assert not kernels.beam_select_supported(lg, sc, 17)  # more than 16 beams
    assert not kernels.beam_select_supported(lg, sc.double(), 5)  # fp64 scores
    assert not kernels.beam_select_supported(torch.zeros(10, 16392, dtype=torch.bfloat16, device=cuda), sc, 5)
    with pytest.raises(ValueError):
        kernels.beam_select(lg, sc, ct, en, 3, False, EOS)  # 10 rows: not groups of 3

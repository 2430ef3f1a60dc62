"""Beam search on bf16 models whose shapes run the MFMA beam kernels: head dim 128 with 8 inputs x 16 heads (the
context by the halves kernel, beams <= 11, after the generated keys' pointer kernel) and head dim 512 (the wide-head
split-K context, the 512-dimension generated-keys kernel, the merge launch).

A bf16 beam search cannot be compared token for token with fp64 on random models: over a search's steps the gaps
between the best offers of different hypotheses fall far below the bf16 error.  What is checked instead:

* one beam is the greedy search: on the margin-filtered fixtures of test_decode_bf16_gpu the beam decoder with one
  beam gives exactly the fp64 reference-order loop's tokens;
* inside a 5-beam search (length normalisation on), the beam attention of the first and the last layer is recorded
  at every step and checked against ``oracle.verify.beam_attention`` on the same inputs (2e-2 abs / 1e-2 rel);
* every step's choice (torch's log-softmax, then the offers and top-k in one launch) equals the choice made on
  torch's own ops over the same logits and state in every group, indices and values bit for bit, with and without
  length normalisation;
* graph replays of the beam step equal eager steps (same tokens, same steps).
"""

import sys

import numpy as np
import pytest
import torch

from oracle import verify as ov
from omniasr_trt_amd import kernels
from omniasr_trt_amd.beam import BeamDecoder

from test_decode_bf16_gpu import shape  # noqa: F401  (the bf16 models and their margin-filtered fixtures)

pytestmark = pytest.mark.gpu
BF16_TOL = (2e-2, 1e-2)


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def npf(t):
    return t.detach().float().cpu().numpy()


def test_one_beam_is_the_greedy_search(shape):  # noqa: F811
    name, m, ctxs, refs = shape
    for graphs in (True, False):
        say(f"{name}: beam decoder, one beam, graphs={graphs}")
        dec = BeamDecoder(m, beams=1, max_batch=8, sync_every=4, reserve=16, graphs=graphs)
        assert dec.generate(ctxs) == refs


def test_beam_attention_inside_the_search(shape, monkeypatch):  # noqa: F811
    name, m, ctxs, refs = shape
    layers = m.dec_cfg.num_layers
    calls, checked = [0], []
    real = kernels.beam_attention

    def recorded(q, kc, vc, ctx_len, kg, vg, ptr, gen_len, beams, ctx_keys, scale, chunk=0, gen_list=None,
                 tickets=None):
        assert gen_list is not None and tickets is not None  # the step's list; the decoder's own tickets
        out = real(q, kc, vc, ctx_len, kg, vg, ptr, gen_len, beams, ctx_keys, scale, chunk, gen_list, tickets)
        i = calls[0] % layers
        calls[0] += 1
        if i in (0, layers - 1) and len(checked) < 24:
            want = ov.beam_attention(npf(q), npf(kc), npf(vc), ctx_len.cpu().numpy(), npf(kg), npf(vg),
                                     ptr.cpu().numpy(), gen_len.cpu().numpy(), beams, scale)
            np.testing.assert_allclose(npf(out), want, atol=BF16_TOL[0], rtol=BF16_TOL[1],
                                       err_msg=f"{name}: beam attention call {calls[0] - 1}")
            checked.append((int(ctx_len.max()), int(gen_len.max())))
        return out

    monkeypatch.setattr(kernels, "beam_attention", recorded)
    dec = BeamDecoder(m, beams=5, length_norm=True, max_batch=8, sync_every=4, reserve=16, graphs=False)
    texts = dec.generate(ctxs)
    say(f"{name}: 5 beams, {len(checked)} beam-attention calls checked (context, generated keys): {checked[:6]} ...")
    assert len(checked) >= 12 and max(g for _, g in checked) >= 3
    assert len(texts) == len(ctxs)


@pytest.mark.parametrize("length_norm", [True, False])
def test_beam_choice_inside_the_search(shape, monkeypatch, length_norm):  # noqa: F811
    """Every step's choice (``kernels.beam_select``: torch's log-softmax, then offers and top-k in one launch) against
    the choice made on torch's own ops (src/omniasr_trt/beam.py:162-175) over the same logits and the search's state
    at that step: identical in every group, indices and values."""
    from test_beam_select_gpu import EOS, choose, torch_offers

    name, m, ctxs, refs = shape
    real = kernels.beam_select
    seen = {"groups": 0, "calls": 0}

    def recorded(logits, score, count, ended, beams, norm, eos, **kw):
        assert not kw.get("fused_log_softmax", False)
        best, flat = real(logits, score, count, ended, beams, norm, eos, **kw)
        assert eos == EOS and norm == length_norm
        rows = logits.size(0)
        offers, _ = torch_offers(logits, score[:rows], count[:rows], ended[:rows], beams, norm)
        want_best, want_flat = choose(offers.view(rows // beams, -1).cpu().numpy(), beams)
        got_best, got_flat = best.cpu().numpy(), flat.cpu().numpy()
        np.testing.assert_array_equal(got_flat, want_flat, err_msg=f"{name}: step {seen['calls']}")
        np.testing.assert_array_equal(got_best, want_best, err_msg=f"{name}: step {seen['calls']}")
        seen["calls"] += 1
        seen["groups"] += len(want_flat)
        return best, flat

    monkeypatch.setattr(kernels, "beam_select", recorded)
    dec = BeamDecoder(m, beams=5, length_norm=length_norm, max_batch=8, sync_every=4, reserve=16, graphs=False)
    texts = dec.generate(ctxs)
    say(f"{name}: length_norm={length_norm}: {seen['calls']} beam steps, all {seen['groups']} group choices "
        f"identical to the choice on torch's offers")
    assert seen["calls"] >= 8
    assert len(texts) == len(ctxs)
    assert int(dec.select_tickets.abs().sum()) == 0


def test_beam_graph_replays_equal_eager_steps(shape):  # noqa: F811
    name, m, ctxs, refs = shape
    a = BeamDecoder(m, beams=5, length_norm=True, max_batch=8, sync_every=4, reserve=16, graphs=True)
    b = BeamDecoder(m, beams=5, length_norm=True, max_batch=8, sync_every=4, reserve=16, graphs=False)
    assert a.generate(ctxs) == b.generate(ctxs)
    assert a.stats["steps"] == b.stats["steps"] and a.stats["captures"] > 0

"""Config 5 (beam variant) at its full shape, step by step: the benchmark's 12-layer stack (d_model 4096, 32 heads x 128,
FFN 11008, vocab 10288, bf16 N(0, 0.02) weights), 8 inputs with contexts of U[750, 2400] random embeddings, 5 beams
each (40 rows), length normalisation on -- the search ``bench.py``'s beam leg times -- run as eager steps with every
kernel's inputs recorded and checked:

* the bookkeeping before the layers (``beam_prepare``) equals ``oracle.verify.beam_prepare`` on the state before the
  step (positions, generated positions, key counts, the rows' own pointers);
* in the first and the last layer, ``beam_attention`` (the context by the halves kernel with the beams as queries,
  the generated keys as tiles of the same launch, each distinct (row, position) once from the step's list) equals
  ``oracle.verify.beam_attention`` on the same inputs within the bf16 bound (2e-2 abs / 1e-2 rel);
* the choice (torch's log-softmax, then the offers and top-k in one launch) equals the choice made on torch's own ops
  over the same logits and state (src/omniasr_trt/beam.py:162-175), indices and values bit for bit;
* the bookkeeping after the top-k (``beam_take_over``) leaves exactly the state ``oracle.verify.beam_take_over``
  computes from the state before it (pointers, histories, scores, counts, flags, tokens, step counters).
"""

import sys

import numpy as np
import pytest
import torch

import bench
from oracle import verify as ov
from omniasr_trt_amd import kernels

from test_beam_select_gpu import choose, torch_offers

pytestmark = pytest.mark.gpu
STEPS = 3
TOL = (2e-2, 1e-2)


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def npf(t):
    return t.detach().float().cpu().numpy()


def host(t):
    return t.detach().cpu().numpy().copy()


def test_config5_beam_steps(cuda, monkeypatch):
    pkg = bench.package()
    say("config 5: the 12-layer bench stack, 8 inputs x 5 beams, length norm")
    with torch.inference_mode():
        model = pkg.modeling.random_decoder(pkg.modeling.BENCH_CONFIG, std=0.02, seed=1004, dtype=torch.bfloat16,
                                            device="cuda")
        dec = pkg.beam.BeamDecoder(model, beams=bench.BEAMS, length_norm=True, max_batch=bench.SLOTS, sync_every=16,
                                   graphs=False)
        rng = np.random.default_rng(1006)
        lengths = rng.integers(750, 2401, bench.SLOTS)
        g = torch.Generator(device="cuda").manual_seed(1006)
        ctxs = [torch.randn(int(n), model.dec_cfg.model_dim, device="cuda", generator=g).to(torch.bfloat16)
                for n in lengths]
        dec.start_groups(ctxs)
        dec.ensure_beam(dec.ccap, STEPS + 4)
    s, n = bench.SLOTS, bench.BEAMS
    r = s * n
    layers = len(dec.layers)
    ckeys = min(dec.ccap, pkg.beam.bucket(int(lengths.max())))
    rec: dict = {}
    real_prepare, real_attn = kernels.beam_prepare, kernels.beam_attention
    real_select, real_take = kernels.beam_select, kernels.beam_take_over

    def prepare(groups, beams, ctx, k_step, group_done, ptr, *out):
        rec["prepare_in"] = (host(ctx[:groups]), host(k_step[:groups]), host(group_done[:groups]), host(ptr))
        real_prepare(groups, beams, ctx, k_step, group_done, ptr, *out)
        rec["prepare_out"] = [host(t) for t in out] + [host(ptr)]

    def attention(q, kc, vc, ctx_len, kg, vg, ptr, gen_len, beams, ctx_keys, scale, chunk=0, gen_list=None,
                  tickets=None):
        assert gen_list is not None and tickets is dec.attn_tickets  # the step's list; the decoder's own tickets
        out = real_attn(q, kc, vc, ctx_len, kg, vg, ptr, gen_len, beams, ctx_keys, scale, chunk, gen_list, tickets)
        i = rec["layer"]
        rec["layer"] += 1
        if i in (0, layers - 1):
            torch.cuda.synchronize()
            gmax = max(int(gen_len.max()), 1)  # the generated positions in use (the oracle reads no others)
            want = ov.beam_attention(npf(q), npf(kc), npf(vc), host(ctx_len), npf(kg[:, :, :gmax]),
                                     npf(vg[:, :, :gmax]), host(ptr)[:, :gmax], host(gen_len), beams, scale)
            np.testing.assert_allclose(npf(out), want, atol=TOL[0], rtol=TOL[1],
                                       err_msg=f"step {rec['step']} layer {i}: beam attention")
            rec["attn_checked"] += 1
        return out

    def select(logits, score, count, ended, beams, norm, eos, **kw):
        best, flat = real_select(logits, score, count, ended, beams, norm, eos, **kw)
        rows = logits.size(0)
        offers, _ = torch_offers(logits, score[:rows], count[:rows], ended[:rows], beams, norm)
        want_best, want_flat = choose(offers.view(rows // beams, -1).cpu().numpy(), beams)
        np.testing.assert_array_equal(host(flat), want_flat, err_msg=f"step {rec['step']}: choice")
        np.testing.assert_array_equal(host(best), want_best, err_msg=f"step {rec['step']}: values")
        return best, flat

    def take_over(best, flat, vocab, ptr, hist, ended, score, count, tok, k_step, group_done, ctx, limit, eos, pad):
        before = [host(t) for t in (ptr, hist, ended, score, count, tok, k_step, group_done)]
        real_take(best, flat, vocab, ptr, hist, ended, score, count, tok, k_step, group_done, ctx, limit, eos, pad)
        o_ptr, o_hist, o_ended, o_score, o_count, o_tok, o_k, o_done = before
        ov.beam_take_over(host(best), host(flat), vocab, o_ptr, o_hist, o_ended, o_score, o_count, o_tok, o_k, o_done,
                          host(ctx), limit, eos, pad)
        for name, got, want in (("ptr", ptr, o_ptr), ("hist", hist, o_hist), ("ended", ended, o_ended),
                                ("score", score, o_score), ("count", count, o_count), ("tok", tok, o_tok),
                                ("k_step", k_step, o_k), ("group_done", group_done, o_done)):
            np.testing.assert_array_equal(host(got), want, err_msg=f"step {rec['step']}: {name}")
        rec["take_checked"] += 1

    monkeypatch.setattr(kernels, "beam_prepare", prepare)
    monkeypatch.setattr(kernels, "beam_attention", attention)
    monkeypatch.setattr(kernels, "beam_select", select)
    monkeypatch.setattr(kernels, "beam_take_over", take_over)
    rec.update(attn_checked=0, take_checked=0)
    with torch.inference_mode():
        for step in range(STEPS):
            rec["step"], rec["layer"] = step, 0
            dec.step_beam(s, ckeys)
            torch.cuda.synchronize()
            ctx, k_step, gdone, ptr = rec["prepare_in"]
            want_ptr = ptr.copy()
            pos, gen_pos, ctx_len, gen_len = ov.beam_prepare(s, n, ctx, k_step, gdone, want_ptr)
            got_pos, got_gen_pos, got_ctx_len, got_gen_len, got_ptr = rec["prepare_out"]
            np.testing.assert_array_equal(got_pos[:r], pos)
            np.testing.assert_array_equal(got_gen_pos[:r], gen_pos)
            np.testing.assert_array_equal(got_ctx_len[:s], ctx_len)
            np.testing.assert_array_equal(got_gen_len[:r], gen_len)
            np.testing.assert_array_equal(got_ptr[:r], want_ptr[:r])
            assert rec["layer"] == layers
            say(f"step {step}: generated keys {gen_len.max()}, scores {host(dec.score[:n]).round(3).tolist()}")
    assert rec["attn_checked"] == 2 * STEPS and rec["take_checked"] == STEPS
    assert int(dec.select_tickets.abs().sum()) == 0 and int(dec.attn_tickets.abs().sum()) == 0
    dec.release()

"""Config 4 at its full shape, step by step: the benchmark's workload (12 layers, d_model 4096, 32 heads x 128, FFN
11008, vocab 10288, bf16, 8 slots with prompts of U[750, 2400] positions and a seeded token history) run as eager
drafted steps, with every kernel's inputs recorded and its effect checked against the oracle:

* the proposal and step assembly (``spec_prepare``) equal ``oracle.verify.spec_prepare`` on the state before the step;
* in the first and the last layer, the rotated q and the K/V rows written equal ``oracle.verify.rope_kv`` of the
  layer's qkv, and every other element of the layer's K/V cache is untouched (the keys below each slot's position
  included);
* the argmax of the verify logits equals the oracle's (``F.log_softmax(...).argmax`` as PyTorch's GPU kernel rounds
  it) on every row whose result does not hinge on the last bits of the log-sum-exp, and the state after acceptance
  equals ``oracle.verify.accept`` applied to the state before: the kept tokens are the argmaxes of the step's own
  logits, and every running slot advances by n + 1 in [1, 5] positions.

Three phases of STEPS steps each, every one from the post-prefill state: own-token drafting from the seeded history
(the benchmark's main leg; the random model's argmax rarely follows a repeat, so about one token per step); perfect
drafts -- the run's own greedy tokens as CTC frames, loaded through ``Row.draft`` and ``SpecDecoder.filled`` -- where
most proposals are kept; and config 5a's drafts, the same frames with 10% of their tokens substituted, where a
proposal is kept up to its first substituted token.  The frames carry enough tokens for every checked step.

The decoder layer math between the kernels (GEMMs, norms) is torch's; what is checked here is the kernels at the
shapes the benchmark times, inside the decoder, with the state they really see."""

import sys

import numpy as np
import pytest
import torch

import bench
from oracle import verify as ov
from omniasr_trt_amd import kernels, spec

pytestmark = pytest.mark.gpu

STEPS = 6


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def npf(t):
    return t.detach().float().cpu().numpy()


def host(t):
    return t.detach().cpu().numpy().copy()


def test_config4_drafted_steps(cuda, monkeypatch):
    pkg = bench.package()
    say("config 4: building the workload (12 layers, 8 slots, U[750, 2400] prompts)")
    with torch.inference_mode():
        w = bench.Workload(pkg, torch)
    dec, b = w.dec, bench.SLOTS
    layers = len(dec.layers)
    watch = {0, layers - 1}
    rec: dict = {}

    real_prepare, real_rope, real_accept = kernels.spec_prepare, kernels.rope_kv, kernels.greedy_accept

    def prepare(*args, **kw):
        res = real_prepare(*args, **kw)
        rec["prepare"] = [t.clone() for t in res]
        return res

    def rope(qkv, cs, pos, k_cache, v_cache, heads, slots=None, cache_pos=None):
        i = len(rec["rope"])
        before = (k_cache.clone(), v_cache.clone()) if i in watch else None
        q = real_rope(qkv, cs, pos, k_cache, v_cache, heads, slots, cache_pos)
        rec["rope"].append(None if before is None else (qkv.clone(), pos.clone(), slots.clone(), q.clone(), before,
                                                        k_cache, v_cache))
        return q

    def accept(logits, tokens, out, tok, last, done, draft_next, start, use_draft, limit, eos, nxt=None):
        rec["logits"] = logits.clone()
        rec["tokens"] = tokens.clone()
        res = real_accept(logits, tokens, out, tok, last, done, draft_next, start, use_draft, limit, eos, nxt)
        rec["nxt"] = res.clone()
        return res

    with torch.inference_mode():
        # perfect drafts for the second phase: the run's own greedy tokens, as CTC frames through Row.draft -> filled
        conts = w.greedy_continuations(8 * STEPS)
        per_segment = pkg.llm.SEGMENT // pkg.llm.HOP
        frames = [pkg.transcribe.frames_from_tokens([c], per_segment, np.random.default_rng(i))
                  for i, c in enumerate(conts)]
        noisy = [pkg.transcribe.frames_from_tokens([c], per_segment, np.random.default_rng(100 + i), substitute=0.1,
                                                   vocab=w.cfg.vocab_size) for i, c in enumerate(conts)]
    say(f"continuation lengths {[len(c) for c in conts]} (a step keeps at most {bench.DRAFT + 1} tokens)")
    assert min(len(c) for c in conts) >= (bench.DRAFT + 1) * STEPS + 1
    monkeypatch.setattr(kernels, "spec_prepare", prepare)
    monkeypatch.setattr(kernels, "rope_kv", rope)
    monkeypatch.setattr(kernels, "greedy_accept", accept)
    cs = npf(dec.m.rope)
    fragile_rows = 0
    accepted = {}
    with torch.inference_mode():
        for phase in ("own tokens", "frame drafts", "substituted frame drafts"):
            if phase != "own tokens":
                w.load_frame_drafts(frames if phase == "frame drafts" else noisy)
            accepted[phase] = 0
            for step in range(STEPS):
                before = {name: host(getattr(dec, name)[:b]) for name in
                          ("out", "draft", "draft_len", "last", "first", "next", "tok", "done", "start")}
                keys = min(dec.capacity, -(-(int(before["last"].max()) + 8 * (bench.DRAFT + 1) + 2) // 256) * 256)
                rec["rope"] = []
                dec.step(b, keys)
                torch.cuda.synchronize()
                say(f"step {step}: keys {keys}, last {before['last'].tolist()}")

                # proposal and step assembly
                tokens, pos, slots, lengths, use, start = ov.spec_prepare(
                    before["out"], before["draft"], before["draft_len"], before["last"], before["first"], before["next"],
                    before["tok"], before["done"], dec.capacity, bench.DRAFT, spec.NGRAM, spec.BEHIND, spec.AHEAD,
                    spec.REACH, 256, 256, spec.SELF_MIN)
                got = [host(t) for t in rec["prepare"]]
                for name, g, want in zip(("tokens", "pos", "slots", "lengths", "use_draft"), got,
                                         (tokens, pos, slots, lengths, use)):
                    np.testing.assert_array_equal(g, want, err_msg=f"step {step}: {name}")
                np.testing.assert_array_equal(host(dec.start[:b]), start)

                # RoPE + append in the watched layers
                assert len(rec["rope"]) == layers
                for i in sorted(watch):
                    qkv, p, sl, q, (k_before, v_before), k_after, v_after = rec["rope"][i]
                    rows = host(sl)
                    cols = host(p)
                    n = len(rows)
                    # the oracle writes token j at column j of a small cache (its K/V rows only)
                    kc = np.zeros((b, dec.heads, n, dec.head_dim), dtype=np.float32)
                    vc = np.zeros_like(kc)
                    want_q = ov.rope_kv(npf(qkv), cs, cols, kc, vc, dec.heads, rows, np.arange(n), "bf16")
                    np.testing.assert_array_equal(npf(q), want_q, err_msg=f"step {step} layer {i}: q")
                    ri, ci = torch.as_tensor(rows, device=cuda), torch.as_tensor(cols, device=cuda)
                    np.testing.assert_array_equal(npf(k_after[ri, :, ci]), kc[rows, :, np.arange(n)])
                    np.testing.assert_array_equal(npf(v_after[ri, :, ci]), vc[rows, :, np.arange(n)])
                    # everything else untouched: put the written rows into the copy taken before, compare all of it
                    k_before[ri, :, ci] = k_after[ri, :, ci]
                    v_before[ri, :, ci] = v_after[ri, :, ci]
                    assert torch.equal(k_before, k_after) and torch.equal(v_before, v_after), f"step {step} layer {i}"
                rec["rope"] = []

                # argmax + acceptance
                logits = npf(rec["logits"])
                nxt = host(rec["nxt"]).reshape(-1)
                want = ov.log_softmax_argmax(logits, "bf16")
                fragile = ov.argmax_is_fragile(logits, "bf16")
                assert not ((nxt != want) & ~fragile).any(), f"step {step}: argmax"
                fragile_rows += int(fragile.sum())
                after = {name: host(getattr(dec, name)[:b]) for name in ("out", "tok", "last", "done", "next")}
                o_out, o_tok, o_last, o_done, o_next = (before[n].copy() for n in ("out", "tok", "last", "done", "next"))
                ov.accept(host(rec["tokens"]), nxt.reshape(b, -1), o_out, o_tok, o_last, o_done, o_next, start, use,
                          pkg.decode.LIMIT, pkg.llm.EOS)
                for name, o in (("out", o_out), ("tok", o_tok), ("last", o_last), ("done", o_done), ("next", o_next)):
                    np.testing.assert_array_equal(after[name], o, err_msg=f"step {step}: {name}")
                advance = after["last"] - before["last"]
                running = ~before["done"]
                assert ((advance[running] >= 1) & (advance[running] <= bench.DRAFT + 1)).all(), advance
                accepted[phase] += int(advance[running].sum())
                say(f"{phase}, step {step}: accepted {advance.tolist()}")
    rows_checked = 3 * STEPS * b * (bench.DRAFT + 1)
    say(f"config 4: {3 * STEPS} steps checked; {fragile_rows} of {rows_checked} argmax rows lse-fragile; tokens accepted "
        f"{accepted}")
    # the greedy run's own tokens as drafts: most proposals are kept (several tokens per row-step); with 10% of them
    # substituted, fewer but still more than one per row-step
    assert accepted["frame drafts"] > 2 * STEPS * b
    assert accepted["substituted frame drafts"] > 1.5 * STEPS * b

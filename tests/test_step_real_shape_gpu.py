"""The drafted step at the real checkpoint's decoder shape (src/omniasr_trt/modeling.py:30-41: 12 layers, d_model
4096, 8 heads x 512, FFN 2816, vocab 10288; random bf16 weights), 8 slots with contexts U[1200, 1700] -- the shape
``bench.py``'s real-shape leg times -- run as eager steps with the kernels' inputs recorded and checked:

* in the first and the last layer, the verify attention (at head dim 512 the balanced wide-head kernel: a fixed
  budget of workgroups per head dealt to the rows by length, merged in the kernel) equals
  ``oracle.verify.verify_attention`` on the same q and caches within the bf16 bound (2e-2 abs / 1e-2 rel), and the
  rotated q and the K/V rows written equal ``oracle.verify.rope_kv`` of the layer's qkv;
* the argmax of the verify logits equals the oracle's on every row not flagged lse-fragile, and the state after
  acceptance equals ``oracle.verify.accept`` applied to the state before.
"""

import sys

import numpy as np
import pytest
import torch

import bench
from oracle import verify as ov
from omniasr_trt_amd import kernels

pytestmark = pytest.mark.gpu

STEPS = 3
TOL = (2e-2, 1e-2)


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def npf(t):
    return t.detach().float().cpu().numpy()


def host(t):
    return t.detach().cpu().numpy().copy()


def test_real_shape_drafted_steps(cuda, monkeypatch):
    pkg = bench.package()
    say("real checkpoint shape: 12 x [4096, 8 x 512, FFN 2816], 8 slots, contexts U[1200, 1700]")
    with torch.inference_mode():
        w = bench.Workload(pkg, torch, seed=1008, cfg=pkg.modeling.DecoderConfig(), lo=1200, hi=1701)
    dec, b = w.dec, bench.SLOTS
    assert (dec.heads, dec.head_dim) == (8, 512)
    layers = len(dec.layers)
    watch = {0, layers - 1}
    rec: dict = {}
    real_rope, real_attn, real_accept = kernels.rope_kv, kernels.draft_attention, kernels.greedy_accept

    def rope(qkv, cs, pos, k_cache, v_cache, heads, slots=None, cache_pos=None):
        q = real_rope(qkv, cs, pos, k_cache, v_cache, heads, slots, cache_pos)
        i = len(rec["rope"])
        rec["rope"].append((qkv.clone(), pos.clone(), slots.clone(), q.clone()) if i in watch else None)
        return q

    def attention(q, k_cache, v_cache, lengths, tokens, keys, scale, **launch):
        out = real_attn(q, k_cache, v_cache, lengths, tokens, keys, scale, **launch)
        i = len(rec["attn"])
        if i in watch:
            torch.cuda.synchronize()
            rows = q.size(0) // tokens
            want = ov.verify_attention(npf(q), npf(k_cache[:rows, :, :keys]), npf(v_cache[:rows, :, :keys]),
                                       host(lengths), tokens, scale)
            np.testing.assert_allclose(npf(out), want, atol=TOL[0], rtol=TOL[1],
                                       err_msg=f"step {rec['step']} layer {i}: verify attention")
            # the keys this step's RoPE wrote into the layer's cache (rows slots, positions pos)
            qkv, pos, slots, qr = rec["rope"][i]
            n = qkv.size(0)
            kc = np.zeros((rows, dec.heads, n, dec.head_dim), dtype=np.float32)
            vc = np.zeros_like(kc)
            want_q = ov.rope_kv(npf(qkv), npf(dec.m.rope), host(pos), kc, vc, dec.heads, host(slots), np.arange(n),
                                "bf16")
            np.testing.assert_array_equal(npf(qr), want_q, err_msg=f"step {rec['step']} layer {i}: q")
            ri, ci = slots.long(), pos.long()
            np.testing.assert_array_equal(npf(k_cache[ri, :, ci]), kc[host(slots), :, np.arange(n)])
            np.testing.assert_array_equal(npf(v_cache[ri, :, ci]), vc[host(slots), :, np.arange(n)])
            rec["checked"] += 1
        rec["attn"].append(None)
        return out

    def accept(logits, tokens, out, tok, last, done, draft_next, start, use_draft, limit, eos, nxt=None):
        rec["logits"], rec["tokens"] = logits.clone(), tokens.clone()
        rec["use"], rec["start"] = host(use_draft), host(start)
        res = real_accept(logits, tokens, out, tok, last, done, draft_next, start, use_draft, limit, eos, nxt)
        rec["nxt"] = res.clone()
        return res

    monkeypatch.setattr(kernels, "rope_kv", rope)
    monkeypatch.setattr(kernels, "draft_attention", attention)
    monkeypatch.setattr(kernels, "greedy_accept", accept)
    rec["checked"] = 0
    fragile_rows = 0
    with torch.inference_mode():
        for step in range(STEPS):
            rec["step"], rec["rope"], rec["attn"] = step, [], []
            before = {name: host(getattr(dec, name)[:b]) for name in ("out", "tok", "last", "done", "next")}
            keys = min(dec.capacity, -(-(int(before["last"].max()) + 8 * (bench.DRAFT + 1) + 2) // 256) * 256)
            dec.step(b, keys)
            torch.cuda.synchronize()
            assert len(rec["attn"]) == layers
            logits = npf(rec["logits"])
            nxt = host(rec["nxt"]).reshape(-1)
            want = ov.log_softmax_argmax(logits, "bf16")
            fragile = ov.argmax_is_fragile(logits, "bf16")
            assert not ((nxt != want) & ~fragile).any(), f"step {step}: argmax"
            fragile_rows += int(fragile.sum())
            after = {name: host(getattr(dec, name)[:b]) for name in ("out", "tok", "last", "done", "next")}
            o_out, o_tok, o_last, o_done, o_next = (before[n].copy() for n in ("out", "tok", "last", "done", "next"))
            ov.accept(host(rec["tokens"]), nxt.reshape(b, -1), o_out, o_tok, o_last, o_done, o_next, rec["start"],
                      rec["use"], pkg.decode.LIMIT, pkg.llm.EOS)
            for name, o in (("out", o_out), ("tok", o_tok), ("last", o_last), ("done", o_done), ("next", o_next)):
                np.testing.assert_array_equal(after[name], o, err_msg=f"step {step}: {name}")
            say(f"step {step}: keys {keys}, advance {(after['last'] - before['last']).tolist()}")
    assert rec["checked"] == 2 * STEPS
    assert int(dec.attn_tickets.abs().sum()) == 0  # the decoder's own merge tickets, left zero
    say(f"real shape: {STEPS} steps, attention and RoPE checked in layers {sorted(watch)}; {fragile_rows} argmax "
        f"rows lse-fragile")
    w.dec.release()

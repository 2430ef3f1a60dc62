"""Benchmark of the MI355X speculative greedy decoder step: verified decoder tokens/s at batch 8, draft 4, and the
verify attention's HBM bandwidth against the roofline.

    python bench.py [--gpus 1] [--steps 64] [--warmup 16]

Workload: a random-init decoder stack (12 layers, d_model 4096, 32 heads x 128, SwiGLU FFN
11008, vocab 10288, bf16 weights N(0, 0.02), EOS suppressed), 8 slots prefilled with random-embedding prompts of
U[750, 2400] tokens whose last 256 positions hold a seeded token history (30% of 3-grams repeated) that the
own-token drafter searches; each slot generates up to 300 tokens.  A *step* is one drafted verify step of the batch
(proposal, 12 x [qkv GEMM, RoPE + KV append, verify attention, output and FFN GEMMs], LM head, argmax +
acceptance), replayed from a HIP graph; the host looks every 8 steps (tokens, finished rows, key bucket), as the
reference's loop does.  ``value``: tokens accepted in the K timed steps / their wall time.

``roofline``: the verify attention (the step's KV-bound kernel) on config 3 -- 8 rows, T = 5, 32 x 128, lengths
U[750, 2400] -- timed with HIP events on the stream it is launched on, over graph replays that cycle through the 12
layers' caches (2.4 GB of K/V: the 256 MB Infinity Cache cannot serve it); achieved = algorithmic bytes / average
launch time.  ``cpu_baseline``: the numpy oracle's drafted step (fp32) on the host cores, on a bounded sample.
"""

from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import platform
import subprocess
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
METRIC = "verified decoder tokens/sec @ batch 8, draft 4; decode-attn HBM GB/s (% peak)"
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
SLOTS, DRAFT, HISTORY, GENERATE = 8, 4, 256, 300


def package():
    sys.path.insert(0, str(ROOT))
    return importlib.import_module("omniasr-trt_amd")


def seeded_history(rng: np.random.Generator, n: int, vocab: int, repeat: float = 0.3) -> list[int]:
    """A token sequence in which about ``repeat`` of the 3-grams repeat an earlier 3-gram."""
    seq: list[int] = []
    while len(seq) < n:
        if len(seq) >= 3 and rng.random() < repeat:
            i = int(rng.integers(0, len(seq) - 2))
            seq += seq[i: i + 3]
        else:
            seq += [int(x) for x in rng.integers(3, vocab, 3)]
    return seq[:n]


def attention_bytes(lengths: np.ndarray, t: int, heads: int, dim: int) -> int:
    """Algorithmic bytes of one verify-attention launch: K and V of the keys the last query of each row sees
    (lengths + t - 1), read once; q read and the output written once (bf16)."""
    keys = int(np.sum(lengths + t - 1))
    return heads * dim * 2 * (2 * keys + 2 * len(lengths) * t)


class Workload:
    """Config 4 on the GPU (or ``cfg`` with contexts U[lo, hi)): the decoder, its drafted decoder, and the
    post-prefill state to start from."""

    def __init__(self, pkg, torch, seed: int = 1004, cfg=None, lo: int = 750, hi: int = 2401):
        self.torch = torch
        m = pkg.modeling
        cfg = m.BENCH_CONFIG if cfg is None else cfg
        self.cfg = cfg
        self.model = m.random_decoder(cfg, std=0.02, seed=seed, dtype=torch.bfloat16, device="cuda")
        with torch.no_grad():
            self.model.final_proj.weight[pkg.llm.EOS].zero_()  # no EOS: every slot generates its budget
        self.dec = pkg.spec.SpecDecoder(self.model, draft_tokens=DRAFT, max_batch=SLOTS, sync_every=8)
        rng = np.random.default_rng(seed)
        self.lengths = rng.integers(lo, hi, SLOTS)
        self.dec.ensure_capacity(int(self.lengths.max()) + GENERATE + 8 * (DRAFT + 1) + 2)
        g = torch.Generator(device="cuda").manual_seed(seed)
        emb = self.model.text_frontend.weight
        ctxs, hist = [], []
        for n in self.lengths:
            h = seeded_history(rng, HISTORY, cfg.vocab_size)
            audio = torch.randn(int(n) - HISTORY, cfg.model_dim, device="cuda", generator=g).to(torch.bfloat16)
            ctxs.append(torch.cat([audio, emb[torch.tensor(h, device="cuda")]]))
            hist.append(h)
        dec, b = self.dec, SLOTS
        with torch.inference_mode():
            first = dec.prefill(ctxs)
        # The slot state after a fill (src/omniasr_trt/decode.py:303-312), with the history as generated tokens:
        # out[t] is the token after position t, so the history's tokens sit at the positions before their own.
        dec.out[:b] = pkg.llm.PAD
        for s, n in enumerate(self.lengths):
            n = int(n)
            dec.out[s, n - HISTORY: n - 1] = torch.tensor(hist[s][1:], device="cuda", dtype=torch.int32)
            dec.out[s, n - 1] = first[s].to(torch.int32)
            dec.first[s] = n - HISTORY  # the own-token search looks back to here
        dec.tok[:b] = first
        dec.last[:b] = torch.tensor(self.lengths - 1, device="cuda")
        dec.done[:b] = False
        dec.draft_len[:b] = 0  # own tokens only (no CTC drafter)
        dec.next[:b] = 1
        self.pkg = pkg
        self.first_history = dec.first[:b].clone()
        self.snapshot = {k: getattr(dec, k)[:b].clone() for k in ("tok", "last", "done", "out", "next", "first",
                                                                    "start", "draft", "draft_len")}
        torch.cuda.synchronize()

    def greedy_continuations(self, steps: int) -> list[list[int]]:
        """Each slot's greedy tokens from the post-prefill state (the first fed token, then what the drafted loop
        accepts in ``steps`` steps), the state restored afterwards."""
        torch, dec, b = self.torch, self.dec, SLOTS
        self.restore()
        self.run(steps)
        last = dec.last[:b].cpu().numpy()
        out = dec.out[:b].cpu().numpy()
        start = self.snapshot["last"].cpu().numpy()
        conts = [[int(x) for x in out[s, start[s]: last[s] + 1]] for s in range(b)]
        self.restore()
        return conts

    def load_frame_drafts(self, frames: list[np.ndarray] | None) -> None:
        """Give every slot a draft the way the transcriber does: per slot CTC frame argmaxes -> ``llm.Row.draft`` of its
        (only) segment -> ``SpecDecoder.drafts`` -> ``SpecDecoder.filled``; ``frames`` None: no drafts (own tokens, the
        seeded history searchable again).  The state after the load becomes the state ``restore`` returns to."""
        pkg, dec, b = self.pkg, self.dec, SLOTS
        self.restore()
        rows = [pkg.llm.Row(index=s, segments=1, frames=None if frames is None else frames[s]) for s in range(b)]
        dec.drafts = lambda j: rows[j].draft(0)
        dec.filled(list(range(b)), list(range(b)))
        dec.drafts = lambda j: None
        if frames is None:
            dec.first[:b] = self.first_history  # the own-token search sees the seeded history again
        self.snapshot = {k: getattr(dec, k)[:b].clone() for k in self.snapshot}
        self.torch.cuda.synchronize()

    def restore(self):
        for k, v in self.snapshot.items():
            getattr(self.dec, k)[:SLOTS].copy_(v)
        self.torch.cuda.synchronize()

    def buckets(self) -> list[int]:
        lo = int(self.lengths.max()) - 1
        hi = lo + GENERATE + 8 * (DRAFT + 1)
        need = [x + 8 * (DRAFT + 1) + 2 for x in (lo, hi)]
        return sorted({min(self.dec.capacity, -(-n // 256) * 256) for n in range(need[0], need[1] + 256, 256)})

    def run(self, steps: int, until_done: bool = False) -> tuple[int, int]:
        """``steps`` drafted steps (``until_done``: until every slot has generated its budget, at most ``steps``) in
        groups of ``sync_every`` replays with a host look after each group; returns (tokens accepted, row-steps of
        running rows).  ``self.steps_run`` holds the steps replayed."""
        torch, dec, b = self.torch, self.dec, SLOTS
        start = self.snapshot["last"].cpu().numpy()
        last = dec.last[:b].cpu().numpy()
        done = dec.done[:b].cpu().numpy()
        tokens = row_steps = 0
        s = 0
        while s < steps and not (until_done and done.all()):
            n = min(dec.sync_every, steps - s)
            need = int(last.max()) + dec.sync_every * dec.step_tokens + 2
            keys = min(dec.capacity, -(-need // 256) * 256)
            run = dec.runner(b, keys)
            for _ in range(n):
                run()
            s += n
            new_last = dec.last[:b].cpu().numpy()
            row_steps += n * int((~done).sum())
            tokens += int((new_last - last).sum())
            last = new_last
            done = dec.done[:b].cpu().numpy()
            over = np.nonzero(~done & (last - start >= GENERATE))[0]
            if len(over):  # the slot's generation budget: finished as the host's repetition stop finishes rows
                dec.done[torch.as_tensor(over, device="cuda")] = True
                done = dec.done[:b].cpu().numpy()
        self.steps_run = s
        return tokens, row_steps


def time_attention(pkg, torch, dec, t: int, reps: int, seed: int = 1003, separate: bool | None = None) -> dict:
    """Config 3 (T = t) timed with HIP events around graph replays of 24 launches cycling through the 12 layers'
    caches."""
    kernels = pkg.kernels
    if separate is None:
        separate = kernels.DRAFT_ATTN["separate"]
    rng = np.random.default_rng(seed)
    lengths = rng.integers(750, 2401, SLOTS)
    keys = -(-(int(lengths.max()) + t) // 256) * 256
    assert keys <= dec.capacity
    heads, dim = dec.heads, dec.head_dim
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(SLOTS * t, heads, dim, device="cuda", generator=g).to(torch.bfloat16)
    lens = torch.tensor(lengths, device="cuda")
    scale = dim ** -0.5
    layers = len(dec.layers)
    launches = 2 * layers
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for i in range(layers):  # warm-up, tickets allocated
            kernels.draft_attention(q, dec.k[i], dec.v[i], lens, t, keys, scale, separate=separate)
        graph = torch.cuda.CUDAGraph()
        graph.capture_begin()
        for j in range(launches):
            kernels.draft_attention(q, dec.k[j % layers], dec.v[j % layers], lens, t, keys, scale, separate=separate)
        graph.capture_end()
        stream.synchronize()
        graph.replay()
        stream.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record(stream)
        for _ in range(reps):
            graph.replay()
        ev1.record(stream)
        stream.synchronize()
    torch.cuda.current_stream().wait_stream(stream)
    us = ev0.elapsed_time(ev1) * 1000.0 / (reps * launches)
    nbytes = attention_bytes(lengths, t, heads, dim)
    flops = 4 * heads * dim * sum(int(n) + i for n in lengths for i in range(t))
    return {"tokens": t, "us": round(us, 2), "bytes": nbytes, "GBps": round(nbytes / us / 1e3, 1),
            "frac_peak": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "TFLOPs": round(flops / us / 1e6, 2),
            "keys": keys, "chunk": kernels.verify_chunk(SLOTS, t, heads, dim, keys), "launches": reps * launches}


def time_small_kernels(pkg, torch, dec, reps: int = 200) -> dict:
    """Config 2 RoPE + append (decode size and the 8 x 2048 prefill size), the causal prefill attention (8 x 2048),
    the fused argmax + acceptance, config 1's verify step (one slot), the proposal, the layers' norm and gate at the step's size and the beam step's
    choice, each timed with HIP events over ``reps`` launches (latency-bound at decode sizes)."""
    kernels, spec = pkg.kernels, pkg.spec
    res = {}
    heads, dim = dec.heads, dec.head_dim
    cs = dec.m.rope
    g = torch.Generator(device="cuda").manual_seed(1002)
    rng = np.random.default_rng(1002)
    kc = torch.zeros(SLOTS, heads, 4096, dim, device="cuda", dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)

    def timed(fn, n):
        """Device time per call: ``n`` calls captured in one graph, replayed between HIP events on the capture stream
        (eager calls would time the host's launch rate for kernels this short)."""
        fn()
        torch.cuda.synchronize()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            fn()
            graph = torch.cuda.CUDAGraph()
            graph.capture_begin()
            for _ in range(n):
                fn()
            graph.capture_end()
            graph.replay()
            stream.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            graph.replay()
            e1.record(stream)
            stream.synchronize()
        torch.cuda.current_stream().wait_stream(stream)
        return e0.elapsed_time(e1) * 1000.0 / n

    for name, tokens_per_slot in (("rope_kv_config2", 5), ("rope_kv_prefill_8x2048", 2048)):
        n = SLOTS * tokens_per_slot
        qkv = torch.randn(n, 3 * heads * dim, device="cuda", generator=g).to(torch.bfloat16)
        if tokens_per_slot == 5:
            base = rng.integers(200, 2001, SLOTS)
            pos = torch.tensor((base[:, None] + np.arange(5)).reshape(-1), device="cuda")
        else:
            pos = torch.arange(2048, device="cuda").repeat(SLOTS)
        slots = torch.arange(SLOTS, device="cuda").repeat_interleave(tokens_per_slot)
        us = timed(lambda: kernels.rope_kv(qkv, cs, pos, kc, vc, heads, slots), reps if n < 1000 else 20)
        nbytes = n * (3 * heads * dim * 2 + dim // 2 * 2 * 4 + 3 * heads * dim * 2 + 16)
        res[name] = {"us": round(us, 2), "bytes": nbytes, "GBps": round(nbytes / us / 1e3, 1)}
    # Causal prefill attention of 8 contexts of 2048 positions over the cache rows just written (MFMA-bound):
    # 4 * D flops per (query, visible key) pair per head.
    width = 2048
    q = torch.randn(SLOTS * width, heads, dim, device="cuda", generator=g).to(torch.bfloat16)
    kc.normal_(generator=g)
    vc.normal_(generator=g)
    rows = torch.arange(SLOTS, device="cuda")
    us = timed(lambda: kernels.prefill_attention(q, kc, vc, rows, width, dim ** -0.5), 10)
    flops = 4 * dim * heads * SLOTS * width * (width + 1) // 2
    res["prefill_attention_8x2048"] = {"us": round(us, 2), "flops": flops, "TFLOPs": round(flops / us / 1e6, 1),
                                       "frac_bf16_peak": round(flops / us / 1e6 / 2500.0, 4)}
    v = dec.m.final_proj.weight.size(0)
    logits = torch.randn(SLOTS * (DRAFT + 1), v, device="cuda", generator=g).to(torch.bfloat16)
    tokens = torch.randint(3, v, (SLOTS, DRAFT + 1), device="cuda", generator=g)
    st = [torch.ones(SLOTS, 4096, device="cuda", dtype=torch.int32), torch.zeros(SLOTS, device="cuda",
                                                                                   dtype=torch.long),
          torch.zeros(SLOTS, device="cuda", dtype=torch.long), torch.ones(SLOTS, device="cuda", dtype=torch.bool)]
    us = timed(lambda: kernels.greedy_accept(logits, tokens, *st, None, None, None, 8188, 2), reps)
    nbytes = logits.numel() * 2
    res["greedy_accept"] = {"us": round(us, 2), "bytes": nbytes, "GBps": round(nbytes / us / 1e3, 1)}
    # Config 1: one slot's verify step, 1 + 4 queries over 1024 prior keys (32 x 128, bf16), then its acceptance
    # over [5, V] logits.
    # 16 disjoint caches (17 MB each) cycled per call, so the 256 MB Infinity Cache cannot serve them.
    t1, n1, sets = DRAFT + 1, 1024, 16
    kv1 = [(torch.randn(1, heads, n1 + 64, dim, device="cuda", generator=g).to(torch.bfloat16),
            torch.randn(1, heads, n1 + 64, dim, device="cuda", generator=g).to(torch.bfloat16)) for _ in range(sets)]
    q1 = torch.randn(t1, heads, dim, device="cuda", generator=g).to(torch.bfloat16)
    len1 = torch.tensor([n1], device="cuda")
    turn = [0]

    def config1_attention():
        kc1, vc1 = kv1[turn[0] % sets]
        turn[0] += 1
        return kernels.draft_attention(q1, kc1, vc1, len1, t1, n1 + t1, dim ** -0.5)

    us_a = timed(config1_attention, reps)
    st1 = [x[:1] for x in st]
    us_g = timed(lambda: kernels.greedy_accept(logits[:t1], tokens[:1], *st1, None, None, None, 8188, 2), reps)
    nbytes = heads * dim * 2 * 2 * (n1 + t1 - 1) + 2 * t1 * heads * dim * 2
    res["config1_verify_step"] = {"attention_us": round(us_a, 2), "attention_bytes": nbytes,
                                  "attention_GBps": round(nbytes / us_a / 1e3, 1),
                                  "greedy_accept_us": round(us_g, 2), "us": round(us_a + us_g, 2)}
    b = SLOTS
    args = (dec.out[:b], dec.draft[:b], dec.draft_len[:b], dec.last[:b], dec.first[:b], dec.next[:b],
            dec.start[:b].clone(), dec.tok[:b], dec.done[:b], dec.capacity, DRAFT, spec.NGRAM, spec.BEHIND,
            spec.AHEAD, spec.REACH, spec.SELF_WINDOW, spec.SELF_MIN)
    us = timed(lambda: kernels.spec_prepare(*args), reps)
    res["spec_prepare"] = {"us": round(us, 2)}
    # The layers' element-wise ops at the step's size (one launch each; torch's ops beside them for reference).
    layer = dec.m.llama_decoder.layers[0]
    cfg = dec.m.dec_cfg
    x = torch.randn(SLOTS * (DRAFT + 1), cfg.model_dim, device="cuda", generator=g).to(torch.bfloat16)
    gi = torch.randn(SLOTS * (DRAFT + 1), 2 * cfg.ffn_dim, device="cuda", generator=g).to(torch.bfloat16)
    norm = layer.self_attn_layer_norm
    gate, inner = gi.chunk(2, -1)
    for name, ours, theirs, nbytes in (
            ("rms_norm_40x4096", lambda: kernels.rms_norm(x, norm.weight, norm.eps), lambda: norm(x),
             x.numel() * 4 + norm.weight.numel() * 2),
            ("silu_mul_40x11008", lambda: kernels.silu_mul(gi), lambda: inner * torch.nn.functional.silu(gate),
             gi.numel() * 3)):
        us, tus = timed(ours, reps), timed(theirs, reps)
        res[name] = {"us": round(us, 2), "bytes": nbytes, "GBps": round(nbytes / us / 1e3, 1),
                     "torch_us": round(tus, 2)}
    # The beam step's choice at config 5b's size (8 inputs x 5 beams): torch's log-softmax and one launch (the
    # default, the reference's choice bit for bit), the log-softmax fused into that launch, and torch's log-softmax,
    # the offers' element-wise ops and topk.
    n, rows, vocab = BEAMS, SLOTS * BEAMS, cfg.vocab_size
    lg = torch.randn(rows, vocab, device="cuda", generator=g).mul_(4).to(torch.bfloat16)
    sc = -torch.rand(rows, device="cuda", generator=g) * 30
    ct = torch.randint(1, 40, (rows,), device="cuda", generator=g)
    en = torch.rand(rows, device="cuda", generator=g) < 0.2

    def torch_select():
        logp = torch.nn.functional.log_softmax(lg, dim=-1)
        lead = ct.view(-1, n)[:, :1].expand(-1, n).reshape(-1, 1)
        c = ct[:, None]
        off = torch.where(lead > 0, (sc[:, None] * c + logp) / (c + 1), sc[:, None] + logp)
        off = off.masked_fill(en[:, None], float("-inf"))
        off[:, 2] = torch.where(en, sc, off[:, 2])
        return off.view(SLOTS, n * vocab).topk(n, dim=-1, sorted=True)

    us = timed(lambda: kernels.beam_select(lg, sc, ct, en, n, True, 2), reps)
    fused = timed(lambda: kernels.beam_select(lg, sc, ct, en, n, True, 2, fused_log_softmax=True), reps)
    res[f"beam_select_{SLOTS}x{n}x{vocab}"] = {"us": round(us, 2), "fused_log_softmax_us": round(fused, 2),
                                                "bytes": lg.numel() * 2, "torch_us": round(timed(torch_select, reps), 2)}
    return res


BEAMS = 5


def beam_attention_bytes(ctx_len: np.ndarray, gen_len: int, rows: int, heads: int, dim: int) -> int:
    """Algorithmic bytes of one beam-attention launch: each input's context K and V read once for all of its beams,
    each row's generated K and V and pointers, q read and the output written (bf16)."""
    ctx = int(np.sum(ctx_len)) * heads * dim * 2 * 2
    gen = rows * gen_len * (heads * dim * 2 * 2 + 4)
    return ctx + gen + 2 * rows * heads * dim * 2


def beam_leg(pkg, torch, w: Workload, steps: int, warmup: int, reps: int) -> dict:
    """Config 5 (beam variant): beam search with 5 beams and length norm over 8 inputs (40 rows) on the bench stack,
    contexts of U[750, 2400] random embeddings.  ``steps`` replays of the step graph after ``warmup`` (host looks
    and repetition checks aside), and the beam attention alone over the 12 layers' caches (HIP events)."""
    beam, kernels = pkg.beam, pkg.kernels
    dec = beam.BeamDecoder(w.model, beams=BEAMS, length_norm=True, max_batch=SLOTS, sync_every=16)
    rng = np.random.default_rng(1006)
    lengths = rng.integers(750, 2401, SLOTS)
    g = torch.Generator(device="cuda").manual_seed(1006)
    ctxs = [torch.randn(int(n), w.cfg.model_dim, device="cuda", generator=g).to(torch.bfloat16) for n in lengths]
    dec.start_groups(ctxs)
    dec.ensure_beam(dec.ccap, warmup + steps + 4)
    ckeys = min(dec.ccap, beam.bucket(int(lengths.max())))
    run = dec.beam_runner(SLOTS, ckeys)
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        run()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    live = int((~dec.gdone[:SLOTS]).sum())
    # The attention alone: the step's shapes (40 rows, generated length 64), 24 launches cycling the 12 layers.
    rows, heads, dim, gen = SLOTS * BEAMS, dec.heads, dec.head_dim, 64
    q = torch.randn(rows, heads, dim, device="cuda", generator=g).to(torch.bfloat16)
    ctx_len = torch.tensor(lengths, device="cuda")
    gen_len = torch.full((rows,), gen, device="cuda", dtype=torch.long)
    ptr = torch.randint(0, rows, (rows, dec.gcap), device="cuda", generator=g, dtype=torch.int32)
    layers = len(dec.layers)
    scale = dim ** -0.5
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        args = lambda i: (q, dec.kc[i], dec.vc[i], ctx_len, dec.kg[i], dec.vg[i], ptr, gen_len, BEAMS, ckeys, scale)
        kernels.beam_attention(*args(0))
        graph = torch.cuda.CUDAGraph()
        graph.capture_begin()
        for j in range(2 * layers):
            kernels.beam_attention(*args(j % layers))
        graph.capture_end()
        graph.replay()
        stream.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            graph.replay()
        e1.record(stream)
        stream.synchronize()
    torch.cuda.current_stream().wait_stream(stream)
    us = e0.elapsed_time(e1) * 1000.0 / (reps * 2 * layers)
    nbytes = beam_attention_bytes(lengths, gen, rows, heads, dim)
    res = {"workload": "config 5b: 5 beams x 8 inputs, length norm, contexts U[750, 2400]", "steps": steps,
           "ms_per_step": round(elapsed * 1e3 / steps, 4),
           "best_beam_tokens_per_s": round(live * steps / elapsed, 2),
           "row_tokens_per_s": round(live * BEAMS * steps / elapsed, 2),
           "attention": {"us": round(us, 2), "bytes": nbytes, "GBps": round(nbytes / us / 1e3, 1),
                         "frac_peak": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "generated_keys": gen,
                         "ctx_keys": ckeys}}
    dec.release()
    return res


def real_shape_step(pkg, torch, steps: int, warmup: int) -> dict:
    """The drafted step at the real checkpoint's decoder shape (src/omniasr_trt/modeling.py:30-41: 12 x [4096,
    8 heads x 512, FFN 2816], vocab 10288; random bf16 weights), 8 slots with contexts U[1200, 1700] -- the shape
    of the only step time the reference publishes (README.md:130: a 5-token step, 8 rows, ~1,450 keys, 2.03 ms on
    an H200 with the trained checkpoint; context, not a comparable target).  Timed like the headline loop."""
    w = Workload(pkg, torch, seed=1008, cfg=pkg.modeling.DecoderConfig(), lo=1200, hi=1701)
    for keys in w.buckets():
        w.dec.runner(SLOTS, keys)
    w.run(warmup)
    w.restore()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    tokens, row_steps = w.run(steps)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    res = {"workload": "real decoder shape: 12 x [4096, 8 x 512, FFN 2816], vocab 10288, 8 slots, contexts "
                       "U[1200, 1700], draft 4 (own tokens)", "steps": steps,
           "ms_per_step": round(elapsed * 1e3 / steps, 4), "tokens_per_s": round(tokens / elapsed, 2),
           "tokens_per_row_step": round(tokens / max(row_steps, 1), 3), "mean_context": float(w.lengths.mean())}
    w.dec.release()
    return res


def time_prefill_real(pkg, torch, caches, width: int = 2048, reps: int = 10) -> dict:
    """The causal prefill of 8 contexts x ``width`` positions at the caches' heads x head dim (the real checkpoint:
    8 x 512), bf16: one launch of the causal kernel per call, three untimed calls first (eager, HIP events); torch's
    fused scaled_dot_product_attention (flash / memory-efficient backends) timed the same way beside it."""
    kernels = pkg.kernels
    heads, dim = caches.heads, caches.head_dim
    g = torch.Generator(device="cuda").manual_seed(1007)
    q = torch.randn(SLOTS * width, heads, dim, device="cuda", generator=g).to(torch.bfloat16)
    rows = torch.arange(SLOTS, device="cuda")
    call = lambda: kernels.prefill_attention(q, caches.k[0], caches.v[0], rows, width, dim ** -0.5)
    for _ in range(3):
        call()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        call()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / reps
    flops = 4 * dim * heads * SLOTS * width * (width + 1) // 2
    res = {"us": round(us, 1), "flops": flops, "TFLOPs": round(flops / us / 1e6, 1),
           "frac_bf16_peak": round(flops / us / 1e6 / 2500.0, 4)}
    # torch's own fused attention on the same q / K / V for comparison: the flash or memory-efficient backend only
    # (the math path is never run: it would materialise the score matrix in bf16 batched products).
    from torch.nn.attention import SDPBackend, sdpa_kernel
    qt = q.view(SLOTS, width, heads, dim).transpose(1, 2)
    kt, vt = caches.k[0][:SLOTS, :, :width], caches.v[0][:SLOTS, :, :width]
    for name, backend in (("flash", SDPBackend.FLASH_ATTENTION), ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
        try:
            with sdpa_kernel([backend]):
                sdpa = lambda: torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, is_causal=True)
                for _ in range(3):
                    sdpa()
                torch.cuda.synchronize()
                e0.record()
                for _ in range(reps):
                    sdpa()
                e1.record()
                torch.cuda.synchronize()
            res[f"torch_sdpa_{name}_us"] = round(e0.elapsed_time(e1) * 1000.0 / reps, 1)
        except RuntimeError as e:  # backend not built for this shape / dtype
            res[f"torch_sdpa_{name}_us"] = None
            res[f"torch_sdpa_{name}_error"] = str(e).splitlines()[0][:120]
    return res


def time_beam_attention(pkg, torch, reps: int, layers: int = 12, seed: int = 1006, heads: int = 32,
                        dim: int = 128) -> dict:
    """Config 5b's beam attention without the decoder: 8 inputs x 5 beams, contexts U[750, 2400] and 64 generated
    keys per row (pointers to random rows), 32 heads x 128 (or ``heads`` x ``dim``), bf16; 12 disjoint cache sets
    cycled (2.6 GB at 32 x 128) so the Infinity Cache cannot serve them; HIP events around graph replays of 24
    launches."""
    kernels = pkg.kernels
    groups, gen, cap, gcap = SLOTS, 64, 2560, 128
    rows = groups * BEAMS
    rng = np.random.default_rng(seed)
    lengths = rng.integers(750, 2401, groups)
    ckeys = -(-int(lengths.max()) // 256) * 256
    g = torch.Generator(device="cuda").manual_seed(seed)
    mk = lambda *shape: torch.randn(*shape, device="cuda", generator=g).to(torch.bfloat16)
    sets = [(mk(groups, heads, cap, dim), mk(groups, heads, cap, dim), mk(rows, heads, gcap, dim),
             mk(rows, heads, gcap, dim)) for _ in range(layers)]
    q = mk(rows, heads, dim)
    ctx_len = torch.tensor(lengths, device="cuda")
    gen_len = torch.full((rows,), gen, device="cuda", dtype=torch.long)
    ptr = torch.randint(0, rows, (rows, gcap), device="cuda", generator=g, dtype=torch.int32)
    scale = dim ** -0.5
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        call = lambda i: kernels.beam_attention(q, *sets[i][:2], ctx_len, *sets[i][2:], ptr, gen_len, BEAMS, ckeys,
                                                scale)
        for i in range(layers):
            call(i)
        graph = torch.cuda.CUDAGraph()
        graph.capture_begin()
        for j in range(2 * layers):
            call(j % layers)
        graph.capture_end()
        graph.replay()
        stream.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            graph.replay()
        e1.record(stream)
        stream.synchronize()
    torch.cuda.current_stream().wait_stream(stream)
    us = e0.elapsed_time(e1) * 1000.0 / (reps * 2 * layers)
    nbytes = beam_attention_bytes(lengths, gen, rows, heads, dim)
    return {"workload": f"config 5b beam attention: 8 inputs x 5 beams, {heads} heads x {dim}, contexts U[750, 2400], "
                        f"64 generated keys",
            "us": round(us, 2), "bytes": nbytes, "GBps": round(nbytes / us / 1e3, 1),
            "frac_peak": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "ctx_keys": ckeys, "launches": reps * 2 * layers}


class AttentionCaches:
    """Config 3 without the decoder: 12 disjoint bf16 K/V sets [8, 32, 2560, 128] (2.5 GB touched per cycle: the
    256 MB Infinity Cache cannot serve them) standing in for the 12 layers' caches; ``heads`` / ``dim`` 8 / 512 give
    the real checkpoint's shape."""

    def __init__(self, torch, layers: int = 12, cap: int = 2560, seed: int = 1005, heads: int = 32, dim: int = 128):
        g = torch.Generator(device="cuda").manual_seed(seed)
        self.k = [torch.randn(SLOTS, heads, cap, dim, device="cuda", generator=g).to(torch.bfloat16)
                  for _ in range(layers)]
        self.v = [torch.randn(SLOTS, heads, cap, dim, device="cuda", generator=g).to(torch.bfloat16)
                  for _ in range(layers)]
        self.layers = [None] * layers
        self.heads, self.head_dim, self.capacity = heads, dim, cap


def copy_reference(torch, nbytes: int = 256 << 20, reps: int = 4) -> dict:
    """A plain device copy of known size (the scale of the HBM byte counters): torch's copy kernel."""
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").random_(0, 255)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000 / reps
    return {"bytes_read": nbytes, "bytes_written": nbytes, "us": round(us, 2), "GBps": round(2 * nbytes / us / 1e3, 1)}


PROFILE = ROOT / "profiles" / "verify_attention_config3.md"


def measured_traffic() -> int | None:
    """HBM bytes per verify-attention launch (main kernel + split merge, config 3, T = 5) from the committed
    rocprofv3 counter summary (FETCH_SIZE and WRITE_SIZE, scaled by a plain copy's counters), or None."""
    try:
        for line in PROFILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def host_cpu() -> tuple[int, str]:
    """The cores this process may run on (``sched_getaffinity``) and the CPU's model name (``lscpu``)."""
    cores = len(os.sched_getaffinity(0))
    model = platform.processor() or "unknown"
    try:
        text = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=30).stdout
        model = next(line.split(":", 1)[1].strip() for line in text.splitlines() if line.startswith("Model name"))
    except Exception:
        pass
    return cores, model


def _median_call(fn, reps: int, budget: float) -> tuple[float, int]:
    """Seconds per call of ``fn``: 1 warm-up call, then the median of at least ``reps`` timed calls (more while
    ``budget`` seconds last)."""
    fn()
    times = []
    t_end = time.perf_counter() + budget
    while len(times) < reps or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if len(times) >= 4 * reps:
            break
    return float(np.median(times)), len(times)


def cpu_configs(pkg, budget: float = 2.0) -> dict:
    """Configs 1-3 on the host cores, per call, with the oracle's numpy kernels (the fp64 attention, the fp32
    log-softmax argmax, the acceptance loop, the RoPE + append): seeded inputs of each config's shape (seed 1000 +
    config), 1 warm-up call, then the median of >= 5 calls."""
    from oracle import verify as ov

    res = {}
    heads, dim, vocab = 32, 128, 10288
    scale = dim ** -0.5
    eos, limit = pkg.llm.EOS, pkg.decode.LIMIT

    def bf16(a):
        return ov.round_to(np.asarray(a, np.float32), "bf16")

    # Config 1: one slot, 1 + 4 queries over 1024 prior keys, then greedy acceptance over [5, V] bf16 logits with a
    # planted argmax matching the first 2 drafts.
    rng = np.random.default_rng(1001)
    t1, n1 = DRAFT + 1, 1024
    q = bf16(rng.standard_normal((t1, heads, dim)))
    kc = bf16(rng.standard_normal((1, heads, n1 + t1, dim)))
    vc = bf16(rng.standard_normal((1, heads, n1 + t1, dim)))
    logits = bf16(rng.standard_normal((t1, vocab)))
    tokens = rng.integers(3, vocab, (1, t1))
    logits[0, tokens[0, 1]] = logits[1, tokens[0, 2]] = 8.0
    lens1 = np.array([n1])

    def config1():
        ov.verify_attention(q, kc, vc, lens1, t1, scale)
        nxt = ov.log_softmax_argmax(logits).reshape(1, t1)
        out = np.zeros((1, 4096), np.int32)
        ov.accept(tokens, nxt, out, np.zeros(1, np.int64), np.array([n1 - 1]), np.zeros(1, bool), None, None, None,
                  limit, eos)

    sec, n = _median_call(config1, 5, budget)
    res["config1_verify_step"] = {"ms_per_call": round(sec * 1e3, 3), "calls": n,
                                  "sample": "attention B=1 T=5 32x128 over 1024 keys (fp64) + log-softmax argmax of "
                                            "[5, 10288] + acceptance"}
    # Config 2: RoPE + KV append, 8 slots x 5 tokens, 32 heads x 128, capacity 4096, positions = lengths U[200, 2000].
    rng = np.random.default_rng(1002)
    cap = 4096
    qkv = bf16(rng.standard_normal((SLOTS * t1, 3 * heads * dim)))
    base = rng.integers(200, 2001, SLOTS)
    pos = (base[:, None] + np.arange(t1)).reshape(-1)
    slots = np.repeat(np.arange(SLOTS), t1)
    cs = ov.rope_table(dim, cap)
    kc2 = np.zeros((SLOTS, heads, cap, dim), np.float32)
    vc2 = np.zeros_like(kc2)
    sec, n = _median_call(lambda: ov.rope_kv(qkv, cs, pos, kc2, vc2, heads, slots), 5, budget)
    res["config2_rope_kv"] = {"ms_per_call": round(sec * 1e3, 3), "calls": n,
                              "sample": "8 slots x 5 tokens, 32 x 128, capacity 4096"}
    del kc2, vc2
    # Config 3: 8 rows, T = 5, lengths U[750, 2400] (the GPU leg's lengths), fp64 attention.
    rng = np.random.default_rng(1003)
    lengths = rng.integers(750, 2401, SLOTS)
    keys = -(-(int(lengths.max()) + t1) // 256) * 256
    q3 = bf16(rng.standard_normal((SLOTS * t1, heads, dim)))
    # One row's worth of keys and values shared by the 8 rows (the oracle converts each row's keys on its own, so the
    # time is a fresh row's; generating 8 distinct rows would only lengthen the set-up).
    kc3 = np.broadcast_to(rng.standard_normal((1, heads, keys, dim), dtype=np.float32), (SLOTS, heads, keys, dim))
    vc3 = np.broadcast_to(rng.standard_normal((1, heads, keys, dim), dtype=np.float32), (SLOTS, heads, keys, dim))
    sec, n = _median_call(lambda: ov.verify_attention(q3, kc3, vc3, lengths, t1, scale), 5, budget)
    nbytes = attention_bytes(lengths, t1, heads, dim)
    res["config3_verify_attention"] = {"ms_per_call": round(sec * 1e3, 3), "calls": n,
                                       "GBps_algorithmic": round(nbytes / sec / 1e9, 2),
                                       "sample": "8 rows x 5 queries, 32 x 128, lengths U[750, 2400] (fp64; "
                                                 "N(0, 1) values, one row's keys shared by the rows)"}
    return res


def cpu_baseline(pkg, torch, w: Workload, seconds: float) -> dict:
    """The numpy oracle's drafted step (fp32) on the host from the same post-prefill state: 1 warm-up step, then
    timed steps for about ``seconds`` (at least 5), its BLAS on every core this process may use; plus configs 1-3
    per call (:func:`cpu_configs`)."""
    from threadpoolctl import threadpool_limits

    from oracle import step as ostep

    spec = pkg.spec
    dec, b = w.dec, SLOTS
    w.restore()
    weights = ostep.weights_from_state_dict(w.model.state_dict())
    cap = dec.capacity
    k = dec.k[:, :b].float().cpu().numpy()
    v = dec.v[:, :b].float().cpu().numpy()
    state = {key: val.cpu().numpy().copy() for key, val in w.snapshot.items()}
    cfg = w.cfg
    npdec = ostep.NumpySpecDecoder(weights, cfg.num_layers, cfg.num_heads, cfg.rms_eps, dec.m.rope.cpu().numpy(), k,
                                   v, state, DRAFT, spec.NGRAM, spec.BEHIND, spec.AHEAD, spec.REACH, spec.SELF_WINDOW,
                                   spec.SELF_MIN, pkg.decode.LIMIT, pkg.llm.EOS)
    cores, model = host_cpu()

    def one_step() -> tuple[int, float]:
        need = int(state["last"].max()) + 8 * (DRAFT + 1) + 2
        keys = min(cap, -(-need // 256) * 256)
        t0 = time.perf_counter()
        got = npdec.step(keys)
        return got, time.perf_counter() - t0

    tokens, times = 0, []
    with threadpool_limits(limits=cores, user_api="blas"):
        one_step()  # warm-up
        t_end = time.perf_counter() + seconds
        while len(times) < 5 or time.perf_counter() < t_end:
            got, dt = one_step()
            tokens += got
            times.append(dt)
        configs = cpu_configs(pkg)
    elapsed = float(np.sum(times))
    return {"value": round(tokens / elapsed, 2), "unit": "verified tokens/s", "cores": cores,
            "kind": "port", "median_step_s": round(float(np.median(times)), 4),
            "sample": f"1 warm-up + {len(times)} drafted steps of config 4 (8 slots x 5 tokens, 12 layers, fp32 numpy "
                      f"oracle, tests/test_oracle_step.py pins it) from the post-prefill state, {elapsed:.1f} s, "
                      f"{tokens} tokens",
            "cpu": model, "configs": configs}


def main() -> int:
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=64)
    p.add_argument("--warmup", type=int, default=16)
    p.add_argument("--attn-reps", type=int, default=20)
    p.add_argument("--cpu-seconds", type=float, default=20.0)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-extra", action="store_true", help="skip the per-kernel figures")
    p.add_argument("--attention-only", action="store_true",
                   help="only the verify attention on config 3 (synthetic caches, no decoder) and a reference copy")
    p.add_argument("--heads", type=int, default=32, help="--attention-only: heads (8 with --head-dim 512: the real "
                   "checkpoint's shape)")
    p.add_argument("--head-dim", type=int, default=128, help="--attention-only: head dim")
    p.add_argument("--beam", action="store_true", help="--attention-only: the beam attention of config 5b instead "
                   "(synthetic caches)")
    p.add_argument("--prefill-only", action="store_true", help="only the causal prefill attention, 8 contexts x 2048 "
                   "positions at 32 x 128 and at the real checkpoint's 8 x 512 (for counter runs)")
    args = p.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every box has one MI355X, and the step shards by slot with no exchange "
              f"(each GPU runs the same kernels on its own slots); --gpus {args.gpus} is not run.", file=sys.stderr)
        return 2
    import torch

    pkg = package()
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X", file=sys.stderr)
        return 2
    if args.prefill_only:
        with torch.inference_mode():
            base = AttentionCaches(torch, layers=1, cap=2048)
            small = time_prefill_real(pkg, torch, base)
            real = time_prefill_real(pkg, torch, AttentionCaches(torch, layers=1, cap=2048, heads=8, dim=512))
        print(json.dumps({"metric": "prefill attention TFLOP/s", "value": real["TFLOPs"], "unit": "TFLOP/s",
                          "n_gpus": 1, "prefill_attention_8x2048x32x128": small,
                          "prefill_attention_real_8x2048x8x512": real}), flush=True)
        return 0
    if args.attention_only and args.beam:
        with torch.inference_mode():
            ref = copy_reference(torch)
            beam = time_beam_attention(pkg, torch, args.attn_reps, heads=args.heads, dim=args.head_dim)
        print(json.dumps({"metric": "beam-attn HBM GB/s (% peak)", "value": beam["GBps"], "unit": "GB/s", "n_gpus": 1,
                          "frac_peak": beam["frac_peak"], "beam_attention": beam, "copy_reference": ref}), flush=True)
        return 0
    if args.attention_only:
        with torch.inference_mode():
            caches = AttentionCaches(torch, heads=args.heads, dim=args.head_dim)
            ref = copy_reference(torch)
            attn = time_attention(pkg, torch, caches, DRAFT + 1, args.attn_reps)
            sweep = [] if args.no_extra else [time_attention(pkg, torch, caches, t, args.attn_reps) for t in (1, 3, 9)]
        print(json.dumps({"metric": "decode-attn HBM GB/s (% peak)", "value": attn["GBps"], "unit": "GB/s",
                          "n_gpus": 1, "frac_peak": attn["frac_peak"], "attention": attn, "attention_sweep": sweep,
                          "copy_reference": ref}), flush=True)
        return 0
    print(f"[bench] building the config-4 workload", file=sys.stderr, flush=True)
    with torch.inference_mode():
        w = Workload(pkg, torch)
        for keys in w.buckets():  # capture every graph the timed steps can need, outside the timed region
            w.dec.runner(SLOTS, keys)
        print(f"[bench] {len(w.dec.graphs)} step graphs captured; warm-up {args.warmup} steps", file=sys.stderr,
              flush=True)
        w.run(args.warmup)
        w.restore()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        tokens, row_steps = w.run(args.steps)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
    print(f"[bench] {args.steps} steps: {tokens} tokens in {elapsed * 1e3:.1f} ms", file=sys.stderr, flush=True)

    ctc = None
    if not args.no_extra:
        # Config 5a: drafts from a synthetic CTC transcript -- the greedy output with 10% of its tokens substituted,
        # laid out as CTC frames -- through Row.draft and SpecDecoder.filled, over every slot's whole budget.
        with torch.inference_mode():
            conts = w.greedy_continuations(GENERATE + 16)
            rng = np.random.default_rng(1005)
            per_segment = pkg.llm.SEGMENT // pkg.llm.HOP
            frames = [pkg.transcribe.frames_from_tokens([c], per_segment, rng, substitute=0.1,
                                                        vocab=w.cfg.vocab_size) for c in conts]
            w.load_frame_drafts(frames)
            w.run(args.warmup)
            w.restore()
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            ctc_tokens, ctc_rows = w.run(10 * GENERATE, until_done=True)
            torch.cuda.synchronize()
            ctc_s = time.perf_counter() - t1
            ctc_steps = w.steps_run
            start = w.snapshot["last"].cpu().numpy()
            out = w.dec.out[:SLOTS].cpu().numpy()
            diverged = []
            for s_, c in enumerate(conts):
                got = out[s_, start[s_]: start[s_] + len(c)]
                diff = np.flatnonzero(got[: len(c)] != np.asarray(c[: len(got)]))
                diverged.append(int(diff[0]) if len(diff) else None)
            w.load_frame_drafts(None)
        ctc = {"workload": "config 5a: CTC frame drafts of the greedy output with 10% substitutions (Row.draft -> "
                           "SpecDecoder.filled), every slot's 300-token budget",
               "steps": ctc_steps, "tokens": ctc_tokens, "tokens_per_s": round(ctc_tokens / ctc_s, 2),
               "ms_per_step": round(ctc_s * 1e3 / max(ctc_steps, 1), 4),
               "tokens_per_row_step": round(ctc_tokens / max(ctc_rows, 1), 3),
               "diverged_at": diverged,
               "note": "diverged_at: per slot, the first generated position where the drafted run's token differs from "
                       "the transcript's source (a greedy run with own-token drafts); after it the draft no longer "
                       "matches and acceptance falls to own-token drafting (bf16 near-ties decided differently by "
                       "steps of other shapes)"}
        print(f"[bench] CTC drafts: {ctc_tokens} tokens in {ctc_steps} steps, {ctc_s * 1e3:.1f} ms, diverged at "
              f"{diverged}", file=sys.stderr, flush=True)
    beams = None
    if not args.no_extra:
        with torch.inference_mode():
            beams = beam_leg(pkg, torch, w, args.steps, args.warmup, args.attn_reps)
        print(f"[bench] beam search: {beams['ms_per_step']} ms/step, attention {beams['attention']['us']} us",
              file=sys.stderr, flush=True)
    real_step = None
    if not args.no_extra:
        with torch.inference_mode():
            real_step = real_shape_step(pkg, torch, args.steps, args.warmup)
        print(f"[bench] real decoder shape (8 x 512 heads, FFN 2816): {real_step['ms_per_step']} ms/step",
              file=sys.stderr, flush=True)
    with torch.inference_mode():
        attn = time_attention(pkg, torch, w.dec, DRAFT + 1, args.attn_reps)
        print(f"[bench] verify attention T=5: {attn['us']} us, {attn['GBps']} GB/s", file=sys.stderr, flush=True)
        sweep = [time_attention(pkg, torch, w.dec, t, args.attn_reps) for t in (1, 3, 9)] if not args.no_extra else []
        extra = time_small_kernels(pkg, torch, w.dec) if not args.no_extra else {}
        if not args.no_extra:  # the real checkpoint's attention shape: 8 heads x 512 (balanced wide-head split-K)
            real = AttentionCaches(torch, heads=8, dim=512)
            extra["verify_attention_real_8x8x512"] = time_attention(pkg, torch, real, DRAFT + 1, args.attn_reps)
            extra["prefill_attention_real_8x2048"] = time_prefill_real(pkg, torch, real)
            del real
        cpu = None
        if not args.no_cpu:
            print(f"[bench] CPU baseline ({args.cpu_seconds:.0f} s)", file=sys.stderr, flush=True)
            cpu = cpu_baseline(pkg, torch, w, args.cpu_seconds)
    line = {
        "metric": METRIC,
        "value": round(tokens / elapsed, 2),
        "unit": "verified tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init bf16 decoder N(0, 0.02), random-embedding prompts, seeded token history",
        "config": {"workload": "config 4: drafted greedy decode loop on the 12-layer 4096/32x128/11008/10288 stack",
                   "slots": SLOTS, "draft_tokens": DRAFT, "prompt_lengths": "U[750, 2400]",
                   "token_budget_per_slot": GENERATE,
                   "timed": f"{args.steps} steps from the post-prefill state (after {args.warmup} warm-up steps)",
                   "drafter": "own tokens (ngram 8, self_min 3: the reference's)",
                   "repetition_stop": "off (EOS suppressed; slots stop at their budget)", "sync_every": 8,
                   "tokens_per_row_step": round(tokens / max(row_steps, 1), 3),
                   "note": "the random model's argmax rarely follows its history, so own-token drafts are rarely "
                           "kept: each step verifies 1 + 4 tokens per slot and keeps about one",
                   "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "kernel": "verify_attn_pair_kernel<128> (config 3, T = 5)",
                     "achieved": attn["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": attn["frac_peak"],
                     "traffic": measured_traffic(), "bytes_per_launch": attn["bytes"], "us_per_launch": attn["us"],
                     "traffic_source": "the committed rocprofv3 FETCH_SIZE + WRITE_SIZE summary of this launch "
                                       "(profiles/verify_attention_config3.md), not measured in this run"},
        "cpu_baseline": cpu,
        "ctc_drafts": ctc,
        "beam_search": beams,
        "step_real_shape": real_step,
        "attention_sweep": sweep,
        "kernels": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

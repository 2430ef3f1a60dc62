"""Batched beam search of the omniASR LLM decoder on MI355X: every input's search as the reference runs it at batch 1.

Rules of the reference's ``BeamDecoder`` (src/omniasr_trt/beam.py) and its batch-1 loop ``beam_reference``
(src/omniasr_trt/llm.py:205-254): an input (a "group" of ``beams`` rows) starts from the ``beams`` best first
tokens; every step each row offers score + log p for every token (``length_norm``: the running mean, switched on
by the group's row 0), a finished row only EOS at its frozen score; the best ``beams`` offers of the group survive
and the rows follow their parents; the repetition stop ends a row at the exact step it fires; the text is row 0's
once every row has finished or the position cap is reached.

Memory layout (HBM):

* ``kc`` / ``vc`` [layers, groups, H, C, Dh]: each input's context, prefilled once and shared by its beams;
* ``kg`` / ``vg`` [layers, rows, H, G, Dh]: the K/V of the token row r fed at generated position j, written once
  at (r, j); ``ptr[r, j]`` (int32) names the row that wrote position j of r's history, so following a parent
  copies pointers and the token history ``hist``, never K/V;
* ``kernels.beam_attention`` reads a group's context once for all of its beams (the verify kernel's MFMA tiles,
  beams as its queries), then each row's generated keys through ``ptr``.

One step (the layers, the LM head, the per-group top-k over beams x vocabulary, the pointer gathers) is one HIP
graph per (groups, context bucket); the host looks every ``sync_every`` steps, or at the exact step a group's
repetition check is due.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import kernels
from .decode import KEY_BUCKET, LIMIT, GreedyDecoder
from .llm import BOS, CHECK_EVERY, CHECK_RATIO, CHECK_WINDOW, EOS, MAX_GEN, PAD, compression_ratio
from .modeling import DecoderModel


def bucket(n: int) -> int:
    """``n`` rounded up to the graph bucket (at least one bucket)."""
    return -(-max(int(n), 1) // KEY_BUCKET) * KEY_BUCKET


class BeamDecoder(GreedyDecoder):
    """Beam search over up to ``max_batch`` inputs at once (``max_batch * beams`` rows).
    (src/omniasr_trt/beam.py:39-59)"""

    def __init__(self, model: DecoderModel, *, beams: int, length_norm: bool = False, max_batch: int = 8,
                 sync_every: int = 16, graphs: bool = True, reserve: int = 512, fused: bool = True):
        if beams < 1 or beams > 16:
            raise ValueError("beams: 1..16")
        super().__init__(model, max_batch=max_batch * beams, sync_every=sync_every, graphs=graphs, reserve=reserve,
                         fused=fused)
        self.beams = beams
        self.length_norm = length_norm
        self.groups = max_batch
        rows, dev = max_batch * beams, self.device
        # Scores as the reference keeps them: fp32, or the model's dtype if that is wider.
        self.score = torch.zeros(rows, device=dev, dtype=torch.promote_types(torch.float32, self.dtype))
        self.ended = torch.ones(rows, device=dev, dtype=torch.bool)
        self.count = torch.zeros(rows, device=dev, dtype=torch.long)  # tokens other than PAD / EOS (length_norm)
        self.rows = torch.arange(rows, device=dev)
        self.group = self.rows // beams
        self.lead = self.group * beams  # row 0 of each row's group
        self.k_step = torch.zeros(max_batch, device=dev, dtype=torch.long)  # tokens chosen in the current context
        self.ctx = torch.ones(max_batch, device=dev, dtype=torch.long)  # its length
        self.gdone = torch.ones(max_batch, device=dev, dtype=torch.bool)
        self.kc = self.vc = self.kg = self.vg = self.ptr = self.hist = None
        self.ccap = self.gcap = 0
        self.stats["repetition_stops"] = 0

    # ------------------------------------------------------------------ buffers

    def ensure_beam(self, ctx_len: int, gen_len: int) -> None:
        """Context caches for ``ctx_len`` positions per input; generated caches, pointers and histories for
        ``gen_len`` positions per row (contents kept when they grow; graphs are captured again)."""
        ctx_len, gen_len = bucket(ctx_len), min(bucket(gen_len), bucket(MAX_GEN))
        if ctx_len <= self.ccap and gen_len <= self.gcap:
            return
        torch.cuda.synchronize(self.device)
        layers, heads, dh, dt, dev = len(self.layers), self.heads, self.head_dim, self.dtype, self.device
        if ctx_len > self.ccap:
            kc = torch.zeros(layers, self.groups, heads, ctx_len, dh, device=dev, dtype=dt)
            vc = torch.zeros_like(kc)
            if self.ccap:
                kc[..., : self.ccap, :] = self.kc
                vc[..., : self.ccap, :] = self.vc
                self.stats["grows"] += 1
            self.kc, self.vc, self.ccap = kc, vc, ctx_len
        if gen_len > self.gcap:
            rows = self.groups * self.beams
            kg = torch.zeros(layers, rows, heads, gen_len, dh, device=dev, dtype=dt)
            vg = torch.zeros_like(kg)
            ptr = torch.zeros(rows, gen_len, device=dev, dtype=torch.int32)
            hist = torch.full((rows, gen_len + 1), PAD, device=dev, dtype=torch.int32)
            if self.gcap:
                kg[..., : self.gcap, :] = self.kg
                vg[..., : self.gcap, :] = self.vg
                ptr[:, : self.gcap] = self.ptr
                hist[:, : self.gcap + 1] = self.hist
                self.stats["grows"] += 1
            self.kg, self.vg, self.ptr, self.hist, self.gcap = kg, vg, ptr, hist, gen_len
        self.reset_graphs()

    def release(self) -> None:
        torch.cuda.synchronize(self.device)
        self.kc = self.vc = self.kg = self.vg = self.ptr = self.hist = None
        self.ccap = self.gcap = 0
        self.reset_graphs()

    # ------------------------------------------------------------------ one step

    def beam_state(self) -> list[torch.Tensor]:
        """What a step changes besides the caches (restored after the warm-up step of a capture)."""
        return [self.tok, self.score, self.ended, self.count, self.k_step, self.gdone, self.hist, self.ptr]

    def step_beam(self, s: int, ckeys: int) -> None:
        """One step of groups 0..s-1 (rows 0..s*N-1), in place; finished groups keep their state.
        (src/omniasr_trt/beam.py:127-187)"""
        m, n = self.m, self.beams
        r = s * n
        tok, score, ended, count = self.tok[:r], self.score[:r], self.ended[:r], self.count[:r]
        k_step, ctx, gdone = self.k_step[:s], self.ctx[:s], self.gdone[:s]
        hist, ptr, rows, group = self.hist[:r], self.ptr[:r], self.rows[:r], self.group[:r]
        live = ~gdone[group]
        k = k_step[group]  # the token in ``tok`` is hist[r, k - 1]
        pos = ctx[group] - 1 + k  # its input position
        j = (k - 1).clamp(min=0)  # its generated cache position
        ctx_len = torch.where(gdone, 0, ctx)
        gen_len = torch.where(live, k, 0)
        # Position j is written by this row in this step, and this step's attention reads it through ``ptr``.
        col = j[:, None]
        ptr.scatter_(1, col, torch.where(live[:, None], rows[:, None].to(ptr.dtype), ptr.gather(1, col)))
        h = m.text_frontend.weight[tok]
        scale = self.head_dim ** -0.5
        for i, layer in enumerate(m.llama_decoder.layers):
            qkv_w, out_w, gi_w, ffo_w = self.layers[i]
            qkv = layer.self_attn_layer_norm(h) @ qkv_w.t()
            q = kernels.rope_kv(qkv, m.rope, pos, self.kg[i], self.vg[i], self.heads, None, j)
            o = kernels.beam_attention(q, self.kc[i], self.vc[i], ctx_len, self.kg[i], self.vg[i], ptr, gen_len, n,
                                       ckeys, scale).reshape(r, -1)
            h.addmm_(o, out_w.t())  # in place: the GEMM adds into the residual, no copy of it
            gate, inner = (layer.ffn_layer_norm(h) @ gi_w.t()).chunk(2, -1)
            h.addmm_(inner * F.silu(gate), ffo_w.t())
        logp = F.log_softmax(m.final_proj(m.llama_decoder.layer_norm(h)), dim=-1)  # [R, V], model dtype
        vocab = logp.size(-1)
        if self.length_norm:
            c = count[:, None]
            mean = (score[:, None] * c + logp) / (c + 1)
            cand = torch.where(count[self.lead[:r]][:, None] > 0, mean, score[:, None] + logp)
        else:
            cand = score[:, None] + logp
        cand = cand.masked_fill(ended[:, None], float("-inf"))
        cand[:, EOS] = torch.where(ended, score, cand[:, EOS])
        top, pick = cand.view(s, n * vocab).topk(n, dim=-1, sorted=True)  # [S, N], best first
        parent = torch.where(live, (pick // vocab + self.lead[:r].view(s, n)[:, :1]).view(-1), rows)
        new = torch.where(live, (pick % vocab).view(-1), tok)
        ptr.copy_(ptr[parent])
        hist.copy_(hist[parent])
        p_ended, p_score, p_count = ended[parent], score[parent], count[parent]
        new = torch.where(p_ended, EOS, new)
        col = k[:, None]
        hist.scatter_(1, col, torch.where(live[:, None], new[:, None].to(hist.dtype), hist.gather(1, col)))
        grows = live & ~p_ended
        score.copy_(torch.where(grows, top.view(-1), p_score))
        count.copy_(p_count + (grows & (new != PAD) & (new != EOS)).long())
        ended.copy_(torch.where(live, new == EOS, p_ended))
        tok.copy_(new)
        k_step.add_((~gdone).long())
        gdone |= ended.view(s, n).all(-1) | (ctx - 2 + k_step >= LIMIT)

    def beam_runner(self, s: int, ckeys: int):
        """The step of groups 0..s-1 with ``ckeys`` context positions in reach: a replayed HIP graph per (s, ckeys)
        (the generated keys' loop bound is read on the device, so it needs no bucket)."""
        if not self.use_graphs:
            return lambda: self.step_beam(s, ckeys)
        key = ("beam", s, ckeys)
        if key not in self.graphs:
            torch.cuda.synchronize(self.device)
            saved = [t.clone() for t in self.beam_state()]
            stream = self.capture_stream
            stream.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(stream):
                self.step_beam(s, ckeys)  # warm-up; the K/V it writes are written again, identically, by the replay
                for t, v in zip(self.beam_state(), saved, strict=True):
                    t.copy_(v)
                graph = torch.cuda.CUDAGraph()
                graph.capture_begin(pool=self.pool)
                self.step_beam(s, ckeys)
                graph.capture_end()
            torch.cuda.current_stream(self.device).wait_stream(stream)
            torch.cuda.synchronize(self.device)
            self.graphs[key] = graph
            self.stats["captures"] += 1
        return self.graphs[key].replay

    # ------------------------------------------------------------------ streams

    @torch.inference_mode()
    def decode_streams(self, n_streams: int, start, advance) -> None:
        """As ``GreedyDecoder.decode_streams``; ``advance(j, tokens)`` receives the best beam's tokens.
        (src/omniasr_trt/beam.py:215-315)"""
        _Groups(self, min(self.groups, n_streams), iter(range(n_streams)), start, advance).run()


class _Groups:
    """Host side of ``BeamDecoder.decode_streams``: the stream each group decodes, the checks due."""

    def __init__(self, dec: BeamDecoder, s: int, upcoming, start, advance):
        self.dec, self.s = dec, s
        self.upcoming, self.start, self.advance = upcoming, start, advance
        self.stream = np.full(s, -1)
        self.ctx_len = np.zeros(s, dtype=np.int64)
        self.normal: tuple[int, int] | None = None

    def fill(self, pairs: list) -> None:
        """Prefill ``pairs`` [(group, stream, context)]; each group starts from its context's N best tokens."""
        dec, n = self.dec, self.dec.beams
        refilled = {g for g, _, _ in pairs}
        k_now = dec.k_step[: self.s].cpu().numpy()
        busy = [int(k_now[g]) for g in range(self.s) if self.stream[g] >= 0 and g not in refilled]
        longest = max(c.size(0) for _, _, c in pairs)
        dec.ensure_beam(max(dec.context_floor, int(self.ctx_len.max()), longest),
                        max([dec.reserve] + [k + dec.sync_every + 2 for k in busy]))
        self.normal = self.normal or (dec.ccap, dec.gcap)
        groups = [g for g, _, _ in pairs]
        with dec.phase("prefill"):
            logp = dec.prefill_into([c for _, _, c in pairs], groups, dec.kc, dec.vc)  # [b, V]
        dec.check("prefill")
        top, first = logp.to(dec.score.dtype).topk(n, dim=-1)  # only one live beam at the first step
        idx = torch.tensor(groups, device=dec.device)
        rows = (idx[:, None] * n + torch.arange(n, device=dec.device)).view(-1)
        first = first.view(-1)
        dec.tok[rows] = first
        dec.score[rows] = top.view(-1)
        dec.ended[rows] = first == EOS
        dec.count[rows] = ((first != PAD) & (first != EOS)).long()
        dec.hist[rows, 0] = first.to(torch.int32)
        lens = torch.tensor([c.size(0) for _, _, c in pairs], device=dec.device)
        dec.k_step[idx] = 1
        dec.ctx[idx] = lens
        dec.gdone[idx] = dec.ended[rows].view(-1, n).all(-1) | (lens - 1 >= LIMIT)
        for g, j, c in pairs:
            self.stream[g], self.ctx_len[g] = j, c.size(0)

    def finish(self, finished: list[int]) -> None:
        dec, n = self.dec, self.dec.beams
        k_now = dec.k_step[: self.s].cpu().numpy()
        hist = dec.hist[: self.s * n].cpu().numpy()
        refill = []
        for g in finished:
            k = int(k_now[g])
            tokens = [int(t) for t in hist[g * n, :k] if t not in (PAD, BOS, EOS)]
            dec.stats["tokens"] += k
            j = int(self.stream[g])
            ctx = self.advance(j, tokens)
            if ctx is None:
                j = next(self.upcoming, None)
                ctx = None if j is None else self.start(j)
            self.stream[g] = -1
            if ctx is not None:
                refill.append((g, j, ctx))
        if refill:
            self.fill(refill)

    def due_step(self, k0: int, c: int) -> int:
        """First k >= k0 at which hist[k] sits at a checked position: c - 1 + k a multiple of ``CHECK_EVERY`` and
        past c + ``CHECK_WINDOW`` (k >= ``CHECK_WINDOW`` + 2)."""
        k = max(k0, CHECK_WINDOW + 2)
        return k + (-(c - 1 + k)) % CHECK_EVERY

    def run(self) -> None:
        dec, s, n = self.dec, self.s, self.dec.beams
        dec.gdone[:s] = True
        dec.k_step[:s] = 1
        dec.tok[: s * n] = 0
        self.fill([(g, j, self.start(j)) for g, j in zip(range(s), self.upcoming)])
        while True:
            gdone = dec.gdone[:s].cpu().numpy()
            finished = [g for g in range(s) if self.stream[g] >= 0 and gdone[g]]
            if finished:
                self.finish(finished)
                continue
            active = [g for g in range(s) if self.stream[g] >= 0]
            if not active:
                break
            k_now = dec.k_step[:s].cpu().numpy()
            # Run up to the step that chooses the token at the next checked position of an active group, so the
            # repetition stop applies exactly there, as in the reference.
            due = {g: self.due_step(int(k_now[g]), int(self.ctx_len[g])) for g in active}
            steps = max(1, min(dec.sync_every, min(due[g] - int(k_now[g]) + 1 for g in active)))
            need = max(int(k_now[g]) for g in active) + steps + 1
            if need + 1 > dec.gcap:
                dec.ensure_beam(dec.ccap, need + dec.reserve)
            ckeys = min(dec.ccap, bucket(max(int(self.ctx_len[g]) for g in active)))
            run = dec.beam_runner(s, ckeys)
            dec.check("runner")
            for _ in range(steps):
                run()
                dec.check("step")
            dec.stats["steps"] += steps
            dec.stats["rows_steps"] += steps * n * len(active)
            k_after = dec.k_step[:s].cpu().numpy()
            checks = [g for g in active if int(k_after[g]) - 1 == due[g]]
            if checks:
                self.repetition_check(checks, due)
        if self.normal is not None and (dec.ccap, dec.gcap) != self.normal:
            dec.release()

    def repetition_check(self, checks: list[int], due: dict) -> None:
        dec, n = self.dec, self.dec.beams
        hist = dec.hist[: self.s * n].cpu().numpy()
        stop = [g * n + b for g in checks for b in range(n)
                if compression_ratio(hist[g * n + b, due[g] - CHECK_WINDOW: due[g]]) > CHECK_RATIO]
        if stop:
            dec.stats["repetition_stops"] += len(stop)
            dec.ended[torch.tensor(stop, device=dec.device)] = True
            groups = torch.tensor(checks, device=dec.device)
            dec.gdone[groups] |= dec.ended[: self.s * n].view(self.s, n)[groups].all(-1)


__all__ = ["BeamDecoder", "bucket"]

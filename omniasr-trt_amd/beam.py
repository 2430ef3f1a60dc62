"""Batched beam search of the omniASR LLM decoder on MI355X: every input's search as the reference runs it at batch 1.

The search of the reference's ``BeamDecoder`` (src/omniasr_trt/beam.py) and of its batch-1 loop ``beam_reference``
(src/omniasr_trt/llm.py:205-254): an input is a *group* of ``beams`` rows that starts from the ``beams`` best first
tokens.  At each step every row offers score + log p for every token (with ``length_norm`` the running mean of its
log-probabilities, used once the group's row 0 has a token), a finished row offers only EOS at its frozen score; the
group keeps its ``beams`` best offers, each row taking over its parent's history; the repetition stop ends a row at
the exact step it fires; the text is row 0's once every row has finished or the position cap is reached.

Memory (HBM):

* ``kc`` / ``vc`` [layers, groups, H, C, Dh]: each input's context, prefilled once for all of its beams;
* ``kg`` / ``vg`` [layers, rows, H, G, Dh]: the K/V of the token row r fed at generated position j, written once at
  (r, j); ``ptr[r, j]`` (int32) names the row whose K/V is position j of r's history, so taking over a parent's
  history copies pointers and token ids (``hist``), never K/V;
* ``kernels.beam_attention`` reads a group's context once for all of its beams (the beams are the queries of the
  verify kernel's tiles), then each row's generated keys through its pointers.

One step (layers, LM head, per-group top-k over beams x vocabulary, the history reorder) is one HIP graph per
(groups, context bucket); the host looks every ``sync_every`` steps, or at the exact step a group's repetition check
is due.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F
from torch import Tensor

from . import kernels
from .batching import UnitScheduler
from .decode import KEY_BUCKET, LIMIT, GreedyDecoder, _regrown
from .llm import BOS, CHECK_EVERY, CHECK_RATIO, CHECK_WINDOW, EOS, MAX_GEN, PAD, compression_ratio
from .modeling import DecoderModel


def bucket(n: int) -> int:
    """``n`` rounded up to the graph bucket, at least one bucket (read at call time, so tests may shrink it)."""
    return -(-max(int(n), 1) // KEY_BUCKET) * KEY_BUCKET


def next_check(k: int, ctx_len: int) -> int:
    """The first step index >= k whose chosen token sits at a checked position: input position ctx_len - 1 + k a
    multiple of ``CHECK_EVERY`` and beyond ctx_len + ``CHECK_WINDOW`` (src/omniasr_trt/llm.py:243-246)."""
    k = max(k, CHECK_WINDOW + 2)
    return k + (-(ctx_len - 1 + k)) % CHECK_EVERY


class BeamDecoder(GreedyDecoder):
    """Beam search over up to ``max_batch`` inputs at once (``max_batch * beams`` rows).
    (src/omniasr_trt/beam.py:39-59)"""

    def __init__(self, model: DecoderModel, *, beams: int, length_norm: bool = False, max_batch: int = 8,
                 sync_every: int = 16, graphs: bool = True, reserve: int = 512, fused: bool = True):
        if not 1 <= beams <= 16:
            raise ValueError("beams: 1..16")
        super().__init__(model, max_batch=max_batch * beams, sync_every=sync_every, graphs=graphs, reserve=reserve,
                         fused=fused)
        self.beams = beams
        self.length_norm = length_norm
        self.groups = max_batch
        rows, dev = max_batch * beams, self.device
        # Row state.  Scores in fp32 as the reference keeps them (fp64 for an fp64 model).
        self.score = torch.zeros(rows, dtype=torch.promote_types(torch.float32, self.dtype), device=dev)
        self.ended = torch.ones(rows, dtype=torch.bool, device=dev)
        # each row's real tokens so far: the length_norm divisor
        self.count = torch.zeros(rows, dtype=torch.long, device=dev)
        # Group state: tokens chosen in the current context, the context's length, finished.
        self.k_step = torch.zeros(max_batch, dtype=torch.long, device=dev)
        self.ctx = torch.ones(max_batch, dtype=torch.long, device=dev)
        self.gdone = torch.ones(max_batch, dtype=torch.bool, device=dev)
        # A step's inputs, rewritten by every step before its layers: rows' input and generated-cache positions,
        # the groups' context key counts, the rows' generated key counts.
        self.row_pos = torch.zeros(rows, dtype=torch.long, device=dev)
        self.gen_pos = torch.zeros(rows, dtype=torch.long, device=dev)
        self.ctx_len = torch.zeros(max_batch, dtype=torch.long, device=dev)
        self.gen_len = torch.zeros(rows, dtype=torch.long, device=dev)
        self.kc = self.vc = self.kg = self.vg = self.ptr = self.hist = None
        self.gen_list = None  # bf16: each group's generated keys once per distinct (row, position), built every step
        self.ccap = self.gcap = 0
        self._normal_caps: tuple[int, int] | None = None
        self.stats["repetition_stops"] = 0
        # This search's own merge tickets of the choice (one per group, zero between launches), so that two searches
        # on different streams of one GPU never share them.
        self.select_tickets = torch.zeros(max_batch, dtype=torch.int32, device=dev)

    # ------------------------------------------------------------------ beam-side cache and search state

    def ensure_beam(self, ctx_len: int, gen_len: int) -> None:
        """Context caches for ``ctx_len`` positions per input, generated caches / pointers / histories for
        ``gen_len`` positions per row (both rounded up to the bucket); growing keeps the contents and drops the
        graphs."""
        want_c, want_g = bucket(ctx_len), min(bucket(gen_len), bucket(MAX_GEN))
        grow_c, grow_g = want_c > self.ccap, want_g > self.gcap
        if not (grow_c or grow_g):
            return
        torch.cuda.synchronize(self.device)
        layers, dev, dt = len(self.layers), self.device, self.dtype
        if grow_c:
            shape = (layers, self.groups, self.heads, want_c, self.head_dim)
            self.kc = _regrown(self.kc, shape, 3, 0, dt, dev)
            self.vc = _regrown(self.vc, shape, 3, 0, dt, dev)
            self.stats["grows"] += bool(self.ccap)
            self.ccap = want_c
        if grow_g:
            rows = self.groups * self.beams
            shape = (layers, rows, self.heads, want_g, self.head_dim)
            self.kg = _regrown(self.kg, shape, 3, 0, dt, dev)
            self.vg = _regrown(self.vg, shape, 3, 0, dt, dev)
            self.ptr = _regrown(self.ptr, (rows, want_g), 1, 0, torch.int32, dev)
            self.hist = _regrown(self.hist, (rows, want_g + 1), 1, PAD, torch.int32, dev)
            if dt == torch.bfloat16:
                self.gen_list = kernels.GenList(self.groups, self.beams, want_g, dev)
            self.stats["grows"] += bool(self.gcap)
            self.gcap = want_g
        self.reset_graphs()

    def release(self) -> None:
        torch.cuda.synchronize(self.device)
        self.kc = self.vc = self.kg = self.vg = self.ptr = self.hist = self.gen_list = None
        self.ccap = self.gcap = 0
        self.reset_graphs()

    # ------------------------------------------------------------------ the search step

    def beam_state(self) -> list[Tensor]:
        """What a step changes besides the caches."""
        return [self.tok, self.score, self.ended, self.count, self.k_step, self.gdone, self.hist, self.ptr]

    def _offers(self, logp: Tensor, r: int) -> Tensor:
        """Every row's offer for every token [R, V]: score + log p (``length_norm``: the mean over the row's tokens,
        once the group's row 0 has one), -inf for a finished row except EOS at its frozen score."""
        score, count, ended = self.score[:r, None], self.count[:r, None], self.ended[:r]
        summed = score + logp
        if self.length_norm:
            lead_count = count.view(-1, self.beams)[:, :1].expand(-1, self.beams).reshape(-1, 1)
            summed = torch.where(lead_count > 0, (score * count + logp) / (count + 1), summed)
        offers = summed.masked_fill(ended[:, None], float("-inf"))
        offers[:, EOS] = torch.where(ended, self.score[:r], offers[:, EOS])
        return offers

    def step_beam(self, s: int, ckeys: int) -> None:
        """One step of groups 0..s-1 (rows 0..s*N-1), in place; finished groups keep their state.  The bookkeeping
        before the layers and after the top-k runs in one launch each (``kernels.beam_prepare`` /
        ``kernels.beam_take_over``), and for bf16 models the log-softmax, offers and top-k in one more
        (``kernels.beam_select``).  (src/omniasr_trt/beam.py:127-187)"""
        n, r = self.beams, s * self.beams
        ptr = self.ptr[:r]
        kernels.beam_prepare(s, n, self.ctx, self.k_step, self.gdone, ptr, self.row_pos, self.gen_pos, self.ctx_len,
                             self.gen_len)
        pos, gen_pos, ctx_len, gen_len = self.row_pos[:r], self.gen_pos[:r], self.ctx_len[:s], self.gen_len[:r]
        lst = self.gen_list
        if lst is not None:  # the beams share most generated keys: list each once for every layer of the step
            kernels.beam_gen_list(lst, ptr, gen_len, self.kg[0], s)
        scale = self.head_dim ** -0.5
        h = self.m.text_frontend.weight[self.tok[:r]]
        for i in range(len(self.layers)):
            kg, vg = self.kg[i], self.vg[i]

            def attend(qkv, i=i, kg=kg, vg=vg):
                q = kernels.rope_kv(qkv, self.m.rope, pos, kg, vg, self.heads, None, gen_pos)
                return kernels.beam_attention(q, self.kc[i], self.vc[i], ctx_len, kg, vg, ptr, gen_len, n, ckeys,
                                              scale, gen_list=lst, tickets=self.attn_tickets).reshape(r, -1)

            self._layer(i, h, attend)
        logits = self._head(h)  # [R, V]
        vocab = logits.size(-1)
        if kernels.beam_select_supported(logits, self.score, n):  # bf16: torch's log-softmax, then offers + top-k
            best, flat = kernels.beam_select(logits, self.score[:r], self.count[:r], self.ended[:r], n,
                                             self.length_norm, EOS, tickets=self.select_tickets)
        else:
            logp = F.log_softmax(logits, dim=-1)  # model dtype
            best, flat = self._offers(logp, r).view(s, n * vocab).topk(n, dim=-1, sorted=True)  # [S, N], best first
        kernels.beam_take_over(best, flat, vocab, ptr, self.hist[:r], self.ended, self.score, self.count, self.tok,
                               self.k_step, self.gdone, self.ctx, LIMIT, EOS, PAD)

    def beam_runner(self, s: int, ckeys: int):
        """The step of groups 0..s-1 with ``ckeys`` context positions in reach, as a callable (a graph replay per
        (s, ckeys); the generated keys' count is read on the device, so it needs no bucket)."""
        before = self.graphs.captures
        run = self.graphs.runner(("beam", s, ckeys), lambda: self.step_beam(s, ckeys), self.beam_state)
        self.stats["captures"] += self.graphs.captures - before
        return run

    # ------------------------------------------------------------------ scheduling beam groups over the inputs

    @torch.inference_mode()
    def decode_streams(self, n_streams: int, start, advance) -> None:
        """As ``GreedyDecoder.decode_streams``; ``advance(j, tokens)`` receives the best beam's tokens.
        (src/omniasr_trt/beam.py:215-315)"""
        s = min(self.groups, n_streams)
        self.gdone[:s] = True
        self.k_step[:s] = 1
        self.tok[: s * self.beams] = 0
        self._normal_caps = None
        UnitScheduler(s, n_streams, start, advance, admit=self.admit,
                      finished=lambda: np.flatnonzero(self.gdone[:s].cpu().numpy()).tolist(),
                      harvest=self._best_tokens, run_block=self._run_block, retire=self._retire).run()

    @torch.inference_mode()
    def start_groups(self, ctxs: list[Tensor]) -> None:
        """Prefill ``ctxs`` into groups 0..len-1 and start their searches, for callers that then drive
        :meth:`beam_runner` by hand (benchmarks)."""
        s = len(ctxs)
        self.gdone[:s] = True
        self.k_step[:s] = 1
        self.tok[: s * self.beams] = 0
        self._normal_caps = None
        sched = UnitScheduler(s, s, ctxs.__getitem__, lambda j, tokens: None, admit=self.admit, finished=list,
                              harvest=self._best_tokens, run_block=lambda sched: None)
        sched.assign([(g, g, c) for g, c in enumerate(ctxs)])

    def admit(self, sched: UnitScheduler, pairs: list) -> None:
        """Prefill ``[(group, stream, context)]`` into their groups' context caches; each group starts from its
        context's ``beams`` most likely first tokens (one live hypothesis at the first step)."""
        n = self.beams
        groups = [g for g, _, _ in pairs]
        ctxs = [c for _, _, c in pairs]
        others = [g for g in sched.active() if g not in set(groups)]
        gen_need = self.reserve
        if others:  # groups still decoding keep room for a whole block of steps
            steps = self.k_step[torch.tensor(others, device=self.device)]
            gen_need = max(gen_need, int(steps.max()) + self.sync_every + 2)
        longest = max(a.ctx_len for a in sched.assigned if a is not None)
        self.ensure_beam(max(self.context_floor, longest), gen_need)
        if self._normal_caps is None:
            self._normal_caps = (self.ccap, self.gcap)
        with self.phase("prefill"):
            logp = self.prefill_into(ctxs, groups, self.kc, self.vc)  # [b, V]
        self.check("prefill")
        top, first = logp.to(self.score.dtype).topk(n, dim=-1)
        idx = torch.tensor(groups, device=self.device)
        rows = (idx[:, None] * n + torch.arange(n, device=self.device)).reshape(-1)
        first = first.reshape(-1)
        self.tok[rows] = first
        self.score[rows] = top.reshape(-1)
        self.ended[rows] = first == EOS
        self.count[rows] = ((first != PAD) & (first != EOS)).long()
        self.hist[rows, 0] = first.to(torch.int32)
        lens = torch.tensor([c.size(0) for c in ctxs], device=self.device)
        self.k_step[idx] = 1
        self.ctx[idx] = lens
        self.gdone[idx] = self.ended[rows].view(-1, n).all(-1) | (lens - 1 >= LIMIT)

    def _best_tokens(self, sched: UnitScheduler, g: int) -> list[int]:
        """Row 0 of a finished group: its tokens of this context (PAD / BOS / EOS dropped)."""
        k = int(self.k_step[g])
        self.stats["tokens"] += k
        return [int(t) for t in self.hist[g * self.beams, :k].tolist() if t not in (PAD, BOS, EOS)]

    def _run_block(self, sched: UnitScheduler) -> None:
        """Replay steps up to the next due repetition check of an active group (at most ``sync_every``), so that the
        check applies exactly at its step, as in the reference; then run the checks that are due."""
        s = sched.units
        active = sched.active()
        k_now = self.k_step[:s].cpu().numpy()
        due = {g: next_check(int(k_now[g]), sched.assigned[g].ctx_len) for g in active}
        steps = max(1, min(self.sync_every, min(due[g] - int(k_now[g]) + 1 for g in active)))
        need = max(int(k_now[g]) for g in active) + steps + 1
        if need + 1 > self.gcap:
            self.ensure_beam(self.ccap, need + self.reserve)
        ckeys = min(self.ccap, bucket(max(sched.assigned[g].ctx_len for g in active)))
        run = self.beam_runner(s, ckeys)
        self.check("runner")
        for _ in range(steps):
            run()
            self.check("step")
        self.stats["steps"] += steps
        self.stats["rows_steps"] += steps * self.beams * len(active)
        k_after = self.k_step[:s].cpu().numpy()
        checks = [g for g in active if int(k_after[g]) - 1 == due[g]]
        if checks:
            self._repetition_stop(checks, due, s)

    def _repetition_stop(self, checks: list[int], due: dict, s: int) -> None:
        """End the rows of ``checks`` whose last ``CHECK_WINDOW`` tokens before their due step compress more than
        ``CHECK_RATIO``; a group whose rows have all ended is done."""
        n = self.beams
        hist = self.hist[: s * n].cpu().numpy()
        stop = [g * n + b for g in checks for b in range(n)
                if compression_ratio(hist[g * n + b, due[g] - CHECK_WINDOW: due[g]]) > CHECK_RATIO]
        if not stop:
            return
        self.stats["repetition_stops"] += len(stop)
        self.ended[torch.tensor(stop, device=self.device)] = True
        groups = torch.tensor(checks, device=self.device)
        self.gdone[groups] |= self.ended[: s * n].view(s, n)[groups].all(-1)

    def _retire(self) -> None:
        if self._normal_caps is not None and (self.ccap, self.gcap) != self._normal_caps:
            self.release()


__all__ = ["BeamDecoder", "bucket", "next_check"]

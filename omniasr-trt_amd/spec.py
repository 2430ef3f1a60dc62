"""Greedy decoding sped up by drafts (speculative decoding), on the MI355X kernels.

The reference's ``SpecDecoder`` (src/omniasr_trt/spec.py): each step feeds a row's newest token and the next
``draft_tokens`` proposed tokens at the positions after it and keeps the proposed tokens the greedy search would
have produced itself (each equal to the argmax after its predecessor) plus the argmax after the last kept one --
1 to ``draft_tokens + 1`` tokens per step, always the greedy search's tokens.  The proposal is searched before
every step in the row's draft (a CTC transcript) around where the previous step left off, and in the row's own
earlier tokens (a repetition loop continued); see ``kernels.propose`` for the rule.

One drafted step here is four kinds of launches around the decoder's GEMMs: ``kernels.spec_prepare`` (proposal
and the step's tokens / positions / key counts), per layer ``kernels.rope_kv`` and ``kernels.draft_attention``
(the T queries of a row share one read of its keys), and ``kernels.greedy_accept`` (argmax of the verify logits,
acceptance, rollback of the cache length).  Rejected drafts' K/V stay in the cache beyond the row's length and
are overwritten by the next step.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import kernels
from .decode import LIMIT, GreedyDecoder  # LIMIT: this module's, read at call time
from .llm import EOS
from .modeling import DecoderModel

# The proposal's search constants (src/omniasr_trt/spec.py:35-40); they decide which tokens are proposed, so they
# are the reference's values.
DRAFT_CAPACITY = 1024  # draft ids held per slot; longer drafts are cut (a 15 s CTC transcript is far shorter)
NGRAM = 8  # how many of a slot's newest tokens a candidate position is matched against
BEHIND, AHEAD = 64, 160  # the draft window around the expected draft position: positions before / after it
# (distance, matches): a draft position at most ``distance`` from the expected one needs ``matches`` leading matches;
# farther positions need NGRAM.  The search cannot jump to a common token far away on a short match.
REACH = ((1, 1), (4, 2), (12, 4), (40, 6))
SELF_WINDOW, SELF_MIN = 256, 3  # own-token search: how far back it looks, and the matches it needs to be used


class SpecDecoder(GreedyDecoder):
    def __init__(self, model: DecoderModel, *, draft_tokens: int = 4, max_batch: int = 8, sync_every: int = 8,
                 ngram: int = NGRAM, self_min: int = SELF_MIN, **options):
        super().__init__(model, max_batch=max_batch, sync_every=sync_every, **options)
        if not 1 <= draft_tokens <= 15:
            raise ValueError("draft_tokens: 1..15 (the verify attention takes up to 16 queries per row)")
        self.draft_tokens = draft_tokens
        self.step_tokens = draft_tokens + 1
        self.ngram, self.self_min = ngram, self_min
        rows, dev = max_batch, self.device
        # Per-slot drafting state, in the layouts the proposal kernel reads: the draft ids (-1 padded) and their
        # count; ``next``, the draft position the search expects to hold the successor of ``tok``; ``first``, the
        # lower bound of the own-token search (the context's last position); ``start``, written by every step, the
        # draft position its proposal was taken from.
        self.draft = torch.full((rows, DRAFT_CAPACITY), -1, device=dev, dtype=torch.int32)
        self.draft_len = torch.zeros(rows, device=dev, dtype=torch.long)
        self.next = torch.zeros(rows, device=dev, dtype=torch.long)
        self.first = torch.zeros(rows, device=dev, dtype=torch.long)
        self.start = torch.zeros(rows, device=dev, dtype=torch.long)
        # Set by the transcriber: stream j -> None or (draft ids, draft position of the context's first generated
        # token) for the stream's current context.
        self.drafts = lambda stream: None

    def state(self) -> list[Tensor]:
        return super().state() + [self.next]

    def filled(self, slots: list[int], streams: list[int]) -> None:
        """Load the draft of each newly filled slot's stream (one host-to-device copy per context, none per step).
        ``drafts(j)`` is None or (ids, where): ``where`` is the draft position of the context's first generated token,
        so the proposal search starts just after it; the own-token search starts at the context's last position.
        (src/omniasr_trt/spec.py:64-74)"""
        for slot, stream in zip(slots, streams, strict=True):
            given = self.drafts(stream)
            ids, where = ([], 0) if given is None else (list(given[0])[:DRAFT_CAPACITY], int(given[1]))
            row = torch.full((DRAFT_CAPACITY,), -1, dtype=torch.int32)
            row[: len(ids)] = torch.as_tensor(ids, dtype=torch.int32)
            self.draft[slot].copy_(row)
            self.draft_len[slot] = len(ids)
            self.next[slot] = where + 1
            self.first[slot] = self.last[slot]

    def propose(self, b: int) -> tuple[Tensor, Tensor]:
        """Per row the next ``draft_tokens`` proposed tokens [B, k] and whether they came from the draft [B].
        (src/omniasr_trt/spec.py:76-80)"""
        return kernels.propose(self.out[:b], self.draft[:b], self.draft_len[:b], self.last[:b], self.first[:b],
                               self.next[:b], self.start[:b], self.draft_tokens, self.ngram, BEHIND, AHEAD, REACH,
                               SELF_WINDOW, self.self_min)

    def step(self, b: int, keys: int) -> None:
        """One drafted step on rows 0..b-1, in place.  (src/omniasr_trt/spec.py:82-108)"""
        k = self.draft_tokens
        tok, last, done, out = self.tok[:b], self.last[:b], self.done[:b], self.out[:b]
        tokens, pos, slots, lengths, use_draft = kernels.spec_prepare(
            out, self.draft[:b], self.draft_len[:b], last, self.first[:b], self.next[:b], self.start[:b], tok, done,
            self.capacity, k, self.ngram, BEHIND, AHEAD, REACH, SELF_WINDOW, self.self_min)
        h = self.m.text_frontend.weight[tokens.view(-1)]  # [B * (k + 1), D]
        logits = self.layer_stack(h, pos, slots, lengths, k + 1, keys)
        kernels.greedy_accept(logits, tokens, out, tok, last, done, self.next[:b], self.start[:b], use_draft,
                              LIMIT, EOS)


__all__ = ["AHEAD", "BEHIND", "DRAFT_CAPACITY", "NGRAM", "REACH", "SELF_MIN", "SELF_WINDOW", "SpecDecoder"]

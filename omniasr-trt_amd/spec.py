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

DRAFT_CAPACITY = 1024  # draft tokens kept per row (a 15 s segment's CTC text is rarely longer than 400)
NGRAM = 8  # newest tokens matched against the draft / the row's own tokens
BEHIND, AHEAD = 64, 160  # draft positions searched before / after the expected one
# Matching tokens a draft position needs at each distance from the expected one (<= 1, <= 4, <= 12, <= 40, beyond).
REACH = ((1, 1), (4, 2), (12, 4), (40, 6))
SELF_WINDOW, SELF_MIN = 256, 3  # own positions searched back, matching tokens needed


class SpecDecoder(GreedyDecoder):
    def __init__(self, model: DecoderModel, *, draft_tokens: int = 4, max_batch: int = 8, sync_every: int = 8,
                 ngram: int = NGRAM, self_min: int = SELF_MIN, **options):
        super().__init__(model, max_batch=max_batch, sync_every=sync_every, **options)
        if not 1 <= draft_tokens <= 15:
            raise ValueError("draft_tokens: 1..15 (the verify attention takes up to 16 queries per row)")
        self.draft_tokens = draft_tokens
        self.step_tokens = draft_tokens + 1
        self.ngram, self.self_min = ngram, self_min
        b, dev = max_batch, self.device
        self.draft = torch.full((b, DRAFT_CAPACITY), -1, device=dev, dtype=torch.int32)
        self.draft_len = torch.zeros(b, device=dev, dtype=torch.long)
        self.next = torch.zeros(b, device=dev, dtype=torch.long)  # draft position expected after ``tok``
        self.first = torch.zeros(b, device=dev, dtype=torch.long)  # position of the segment's first token
        self.start = torch.zeros(b, device=dev, dtype=torch.long)  # draft position of a step's first proposal
        # The transcriber's: a stream's draft for its current context, (token ids, draft position of the first
        # generated token), or None.
        self.drafts = lambda stream: None

    def state(self) -> list[Tensor]:
        return super().state() + [self.next]

    def filled(self, slots: list[int], streams: list[int]) -> None:
        """Load each refilled slot's draft (one host-to-device copy per slot fill, not per step).
        (src/omniasr_trt/spec.py:64-74)"""
        for s, j in zip(slots, streams, strict=True):
            draft = self.drafts(j)
            tokens, start = draft if draft is not None else ([], 0)
            tokens = list(tokens)[:DRAFT_CAPACITY]
            self.draft[s] = -1
            if tokens:
                self.draft[s, : len(tokens)] = torch.as_tensor(tokens, dtype=torch.int32).to(self.device)
            self.draft_len[s] = len(tokens)
            self.next[s] = start + 1
            self.first[s] = self.last[s]

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

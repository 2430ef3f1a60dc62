"""The decoder side of omniASR-LLM's streaming transcription: segment contexts, the choice of decoder, and CTC-frame
drafts fed to the drafted decoder.

What the reference's ``LLMTranscriber`` does between its audio encoder and its tokenizer
(src/omniasr_trt/llm.py:88-340), on audio that is already embedded: an input is cut into 15 s segments, and segment
i is decoded with segment i-1's audio and text as its context,

    [lang] <lid> (audio_{i-1} <regular> <bos> text_{i-1} <eos>) audio_i <last|regular> <bos> -> text_i <eos>

(src/omniasr_trt/llm.py:160-173); every input's segments run one after another as one stream of the decoder, and the
inputs share the decoder's slots.  With ``draft_tokens`` > 0 the greedy search is the drafted decoder, and each
segment's draft is the CTC transcript of its frames and a margin around them (:meth:`llm.Row.draft`), handed to the
decoder through its ``drafts`` callback when the segment's context is admitted (src/omniasr_trt/llm.py:315-340).

The encoder (wav2vec2 + projection), the CTC model and the tokenizer are not part of the decode step and are not
here: an input is given as its segments' decoder embeddings ``[F_i, model_dim]``, a drafter as an object with
``frame_ids(audio) -> per input CTC argmax of each 20 ms frame``, and the result is token ids (or text, with a
tokenizer that has ``decode(ids)``).
"""

from __future__ import annotations

import time
from contextlib import contextmanager

import numpy as np
import torch
from torch import Tensor

from .beam import BeamDecoder
from .decode import GreedyDecoder
from .llm import BOS, EOS, PAD, Row, as_frames
from .modeling import DecoderModel
from .spec import SpecDecoder


class Transcriber:
    """Streaming transcription of embedded audio with the MI355X decoders; the reference's ``LLMTranscriber``
    constructor options that concern decoding (src/omniasr_trt/llm.py:88-109)."""

    def __init__(self, model: DecoderModel, tokenizer=None, *, max_batch: int = 8, reserve: int = 512, beams: int = 1,
                 length_norm: bool = False, drafter=None, draft_tokens: int = 4):
        self.model = model
        self.tokenizer = tokenizer
        self.max_batch = max_batch
        self.reserve = reserve
        self.beams, self.length_norm = beams, length_norm  # search defaults (beams 1: greedy)
        self.drafter = drafter  # None: the drafted search proposes from each row's own tokens only
        self.draft_tokens = draft_tokens  # tokens proposed per drafted step (0: one token per step)
        vocab = model.dec_cfg.vocab_size
        self.lid, self.last_seg, self.regular_seg = vocab, vocab + 1, vocab + 2  # special text embedding rows
        self.dtype = model.final_proj.weight.dtype
        self.device = model.final_proj.weight.device
        self._decoders: dict = {}
        self.last_decoder = None
        self.profile = False  # True: each phase synchronises the device and adds its seconds to ``timings``
        self.timings: dict[str, float] = {}

    @contextmanager
    def phase(self, name: str):
        if not self.profile:
            yield
            return
        torch.cuda.synchronize(self.device)
        t0 = time.perf_counter()
        try:
            yield
        finally:
            torch.cuda.synchronize(self.device)
            self.timings[name] = self.timings.get(name, 0.0) + time.perf_counter() - t0

    # ------------------------------------------------------------------ audio segments and prompts

    def rows(self, audio: list, langs=None, drafts=None) -> list[Row]:
        """One :class:`Row` per input: ``audio[j]`` the list of its segments' embeddings, ``langs[j]`` its language
        embedding row (None: 0), ``drafts[j]`` its CTC frame argmaxes (None: no draft)."""
        langs = [None] * len(audio) if langs is None else list(langs)
        drafts = [None] * len(audio) if drafts is None else list(drafts)
        if not len(audio) == len(langs) == len(drafts):
            raise ValueError("audio, langs and drafts: one entry per input")
        out = []
        for j, (segs, lang, frames) in enumerate(zip(audio, langs, drafts)):
            segs = [s.to(self.device, self.dtype) for s in segs]
            if not segs:
                raise ValueError(f"input {j}: no segment")
            out.append(Row(index=j, segments=len(segs), lang=0 if lang is None else int(lang), audio=segs,
                           frames=as_frames(frames)))
        return out

    def context(self, r: Row, i: int) -> Tensor:
        """Decoder input embeddings ``[C, D]`` of segment ``i`` of row ``r``, ending with <bos>
        (src/omniasr_trt/llm.py:160-173)."""
        text = self.model.text_frontend.weight

        def ids(values: list[int]) -> Tensor:
            return text[torch.tensor(values, dtype=torch.long, device=self.device)]

        pieces = [self.model.lang_embeddings.weight[r.lang: r.lang + 1], ids([self.lid])]
        if i > 0:  # the previous segment, audio and text, as context
            pieces += [r.audio[i - 1], ids([self.regular_seg, BOS, *r.tokens[i - 1], EOS])]
        marker = self.last_seg if i == r.segments - 1 else self.regular_seg
        pieces += [r.audio[i], ids([marker, BOS])]
        return torch.cat([p.to(self.dtype) for p in pieces])

    def text(self, r: Row):
        ids = [t for seg in r.tokens for t in seg if t not in (PAD, BOS, EOS)]
        return ids if self.tokenizer is None else self.tokenizer.decode(ids)

    # ------------------------------------------------------------------ decoding

    def decoder(self, beams: int, length_norm: bool):
        """The decoder for this search, one kept per setting (the others' caches are released): the drafted decoder
        for greedy search with ``draft_tokens`` > 0, the one-token greedy decoder with 0, beam search otherwise.
        (src/omniasr_trt/llm.py:284-313)"""
        greedy = beams == 1 and not length_norm
        if greedy:
            key = ("spec", self.draft_tokens) if self.draft_tokens > 0 else ("greedy",)
        else:
            key = ("beam", beams, length_norm)
        dec = self._decoders.get(key)
        if dec is None:
            if key[0] == "spec":
                dec = SpecDecoder(self.model, draft_tokens=self.draft_tokens, max_batch=self.max_batch,
                                  reserve=self.reserve)
            elif key[0] == "greedy":
                dec = GreedyDecoder(self.model, max_batch=self.max_batch, reserve=self.reserve)
            else:
                dec = BeamDecoder(self.model, beams=beams, length_norm=length_norm, max_batch=self.max_batch,
                                  reserve=self.reserve)
            self._decoders[key] = dec
        for other_key, other in self._decoders.items():
            if other_key != key and (getattr(other, "capacity", 0) or getattr(other, "ccap", 0)):
                other.release()
        dec.phase = self.phase
        self.last_decoder = dec
        return dec

    def transcribe_rows(self, rows: list[Row], beams: int = 1, length_norm: bool = False) -> list:
        """Decode every segment of every row: each row is one stream of contexts (segment i + 1's context holds
        segment i's tokens), the rows share the decoder's slots.  The drafted decoder takes each segment's draft from
        the row's CTC frames when the segment is admitted.  (src/omniasr_trt/llm.py:315-340)"""
        dec = self.decoder(beams, length_norm)
        drafted = isinstance(dec, SpecDecoder)
        if drafted:
            dec.drafts = lambda j: rows[j].draft(len(rows[j].tokens))

        def first_context(j: int) -> Tensor:
            with self.phase("context"):
                return self.context(rows[j], 0)

        def next_context(j: int, tokens: list[int]) -> Tensor | None:
            r = rows[j]
            r.tokens.append(tokens)
            if len(r.tokens) == r.segments:
                return None
            with self.phase("context"):
                return self.context(r, len(r.tokens))

        try:
            with self.phase("decoder"):
                dec.decode_streams(len(rows), first_context, next_context)
        finally:
            if drafted:
                dec.drafts = lambda j: None  # the rows (their embeddings) are not held after the call
        return [self.text(r) for r in rows]

    @torch.inference_mode()
    def transcribe(self, audio: list, langs=None, *, mode: str = "fast", beams: int | None = None,
                   length_norm: bool | None = None, drafts=None) -> list:
        """Token ids (or texts, with a tokenizer) of each input.  ``beams`` / ``length_norm``: the search (default: the
        transcriber's).  ``drafts``: per input the CTC argmax of each 20 ms frame (default: the drafter's, if any),
        used by the greedy search only.  ``mode``: "fast" (the batched decoders on the MI355X kernels); the
        reference's "reference" mode -- its batch-1 torch loops -- is not a path of this package and is refused.
        (src/omniasr_trt/llm.py:255-282)"""
        if mode != "fast":
            raise ValueError(f"mode={mode!r}: only 'fast' (the batched MI355X decoders); the reference's batch-1 "
                             "'reference' loops are not part of this package")
        beams = self.beams if beams is None else beams
        length_norm = self.length_norm if length_norm is None else length_norm
        greedy = beams == 1 and not length_norm
        if drafts is None and self.drafter is not None and greedy and self.draft_tokens:
            with self.phase("drafter"):
                drafts = self.drafter.frame_ids(audio)
        rows = self.rows(audio, langs, drafts if greedy else None)
        return self.transcribe_rows(rows, beams, length_norm)


def frames_from_tokens(segments: list[list[int]], frames_per_segment: int, rng: np.random.Generator,
                       substitute: float = 0.0, vocab: int | None = None) -> np.ndarray:
    """A synthetic CTC frame sequence whose segment i carries ``segments[i]``: within each segment's frames the tokens
    in order, each followed by a blank (id 0) and held for a second frame where the segment has room for it, then
    blanks (a segment with fewer than two frames per token gets its tokens back to back, cut at its end); with
    ``substitute`` > 0 each token is replaced by a random id in [3, vocab) with that probability (the config-5a
    drafter).  For benchmarks and tests: a stand-in for an omniASR CTC model's ``frame_ids``."""
    out = np.zeros(frames_per_segment * len(segments), dtype=np.int64)
    for i, toks in enumerate(segments):
        toks = [int(rng.integers(3, vocab)) if substitute and rng.random() < substitute else int(t) for t in toks]
        pos, end = i * frames_per_segment, (i + 1) * frames_per_segment
        spaced = 2 * len(toks) <= frames_per_segment
        for n, t in enumerate(toks):
            if pos >= end:
                break
            spare = end - pos - 2 * (len(toks) - n)  # frames beyond one token + one blank for every token left
            hold = 2 if spaced and spare > 0 and rng.random() < 0.5 else 1
            out[pos: pos + hold] = t
            pos += hold + (1 if spaced else 0)
    return out


__all__ = ["Transcriber", "frames_from_tokens"]

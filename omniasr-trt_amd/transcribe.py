"""The decoder side of omniASR-LLM's streaming transcription: segment prompts, the choice of decoder, and CTC-frame
drafts fed to the drafted decoder.

What the reference's ``LLMTranscriber`` does between its audio encoder and its tokenizer
(src/omniasr_trt/llm.py:88-340), on audio that is already embedded.  An input is cut into 15 s segments, and
segment i is decoded with segment i-1's audio and text in its prompt,

    [lang] <lid> (audio_{i-1} <regular> <bos> text_{i-1} <eos>) audio_i <last|regular> <bos> -> text_i <eos>

(src/omniasr_trt/llm.py:160-173).  Every input's segments run one after another as one stream of the decoder, and
the inputs share the decoder's slots.  With ``draft_tokens`` > 0 the greedy search is the drafted decoder, and each
segment's draft is the CTC transcript of its frames and a margin around them (:meth:`llm.Row.draft`), handed to the
decoder through its ``drafts`` callback when the segment is admitted (src/omniasr_trt/llm.py:315-340).

The encoder (wav2vec2 + projection), the CTC model and the tokenizer are not part of the decode step and are not
here: an input is given as its segments' decoder embeddings ``[F_i, model_dim]``, a drafter as an object with
``frame_ids(audio) -> per input CTC argmax of each 20 ms frame``, and the result is token ids (or text, with a
tokenizer that has ``decode(ids)``).

Three parts: :class:`PromptLayout` states the prompt above as data, :class:`DecoderPool` keeps one decoder per search
setting (only the one in use holds caches), and :class:`SegmentStreams` feeds a decoder's stream callbacks from the
inputs' segments.  :class:`Transcriber` puts them together.
"""

from __future__ import annotations

import time
from contextlib import contextmanager, nullcontext

import numpy as np
import torch
from torch import Tensor

from .beam import BeamDecoder
from .decode import GreedyDecoder
from .llm import BOS, EOS, PAD, Row, as_frames
from .modeling import DecoderModel
from .spec import SpecDecoder


class PromptLayout:
    """The decoder prompt of segment i of an input (src/omniasr_trt/llm.py:160-173), built from a list of parts: an
    embedding row range, a run of text token ids, or audio embeddings.  The special ids follow the text vocabulary:
    <lid>, <last segment>, <regular segment>."""

    def __init__(self, model: DecoderModel, dtype: torch.dtype, device: torch.device):
        self.model, self.dtype, self.device = model, dtype, device
        vocab = model.dec_cfg.vocab_size
        self.lid, self.last_seg, self.regular_seg = vocab, vocab + 1, vocab + 2

    def parts(self, row: Row, i: int) -> list[tuple[str, object]]:
        """(kind, value) parts in prompt order: "lang" (a language embedding row), "ids" (text ids), "audio"."""
        closing = self.last_seg if i == row.segments - 1 else self.regular_seg
        history = [("audio", row.audio[i - 1]), ("ids", [self.regular_seg, BOS, *row.tokens[i - 1], EOS])] if i else []
        return [("lang", row.lang), ("ids", [self.lid]), *history, ("audio", row.audio[i]), ("ids", [closing, BOS])]

    def embed(self, parts: list[tuple[str, object]]) -> Tensor:
        """The parts' embeddings ``[C, D]`` in the model's dtype."""
        rows = []
        for kind, value in parts:
            if kind == "lang":
                rows.append(self.model.lang_embeddings.weight[value: value + 1])
            elif kind == "ids":
                rows.append(self.model.text_frontend.weight[torch.tensor(value, dtype=torch.long, device=self.device)])
            else:
                rows.append(value)
        return torch.cat([r.to(self.dtype) for r in rows])

    def __call__(self, row: Row, i: int) -> Tensor:
        return self.embed(self.parts(row, i))


def search_key(beams: int, length_norm: bool, draft_tokens: int) -> tuple:
    """The decoder a search runs on (src/omniasr_trt/llm.py:284-313): beam search unless it is one beam without length
    normalisation; then the drafted greedy decoder with ``draft_tokens`` > 0, the one-token greedy decoder with 0."""
    if beams != 1 or length_norm:
        return ("beam", beams, length_norm)
    return ("spec", draft_tokens) if draft_tokens > 0 else ("greedy",)


class DecoderPool:
    """One decoder per search key, built on first use; taking one releases the caches of every other, so only the
    decoder in use holds device memory."""

    def __init__(self, model: DecoderModel, max_batch: int, reserve: int):
        self.model, self.max_batch, self.reserve = model, max_batch, reserve
        self.decoders: dict[tuple, object] = {}

    def _build(self, key: tuple):
        kind = key[0]
        if kind == "spec":
            return SpecDecoder(self.model, draft_tokens=key[1], max_batch=self.max_batch, reserve=self.reserve)
        if kind == "greedy":
            return GreedyDecoder(self.model, max_batch=self.max_batch, reserve=self.reserve)
        return BeamDecoder(self.model, beams=key[1], length_norm=key[2], max_batch=self.max_batch,
                           reserve=self.reserve)

    def take(self, key: tuple):
        dec = self.decoders.get(key)
        if dec is None:
            dec = self.decoders[key] = self._build(key)
        for other_key, other in self.decoders.items():
            holds = getattr(other, "capacity", 0) or getattr(other, "ccap", 0)
            if other_key != key and holds:
                other.release()
        return dec


class SegmentStreams:
    """The stream callbacks of ``decode_streams`` over the inputs' rows: stream j opens with segment 0's prompt, and
    each finished segment's tokens go into the row and yield the next segment's prompt (None after the last)."""

    def __init__(self, rows: list[Row], prompt, timed):
        self.rows, self.prompt, self.timed = rows, prompt, timed

    def first(self, j: int) -> Tensor:
        with self.timed("context"):
            return self.prompt(self.rows[j], 0)

    def advance(self, j: int, tokens: list[int]) -> Tensor | None:
        row = self.rows[j]
        row.tokens.append(tokens)
        if len(row.tokens) == row.segments:
            return None
        with self.timed("context"):
            return self.prompt(row, len(row.tokens))

    def draft(self, j: int):
        """The CTC draft of stream j's segment now being admitted (the segment after its finished ones)."""
        row = self.rows[j]
        return row.draft(len(row.tokens))


class Transcriber:
    """Streaming transcription of embedded audio with the MI355X decoders, taking the reference's ``LLMTranscriber``
    constructor options that concern decoding (src/omniasr_trt/llm.py:88-109)."""

    def __init__(self, model: DecoderModel, tokenizer=None, *, max_batch: int = 8, reserve: int = 512, beams: int = 1,
                 length_norm: bool = False, drafter=None, draft_tokens: int = 4):
        self.model = model
        self.tokenizer = tokenizer
        self.beams, self.length_norm = beams, length_norm  # search defaults (beams 1: greedy)
        self.drafter = drafter  # None: the drafted search proposes from each row's own tokens only
        self.draft_tokens = draft_tokens  # tokens proposed per drafted step (0: one token per step)
        weight = model.final_proj.weight
        self.layout = PromptLayout(model, weight.dtype, weight.device)
        self.pool = DecoderPool(model, max_batch, reserve)
        self.last_decoder = None
        self.profile = False  # True: each named phase synchronises the device and adds its seconds to ``timings``
        self.timings: dict[str, float] = {}

    @property
    def device(self) -> torch.device:
        return self.layout.device

    def timed(self, name: str):
        """A context manager around one named phase: a no-op unless ``profile`` is set."""
        return self._timed(name) if self.profile else nullcontext()

    @contextmanager
    def _timed(self, name: str):
        torch.cuda.synchronize(self.device)
        start = time.perf_counter()
        try:
            yield
        finally:
            torch.cuda.synchronize(self.device)
            self.timings[name] = self.timings.get(name, 0.0) + time.perf_counter() - start

    # ------------------------------------------------------------------ inputs and outputs

    def rows(self, audio: list, langs=None, drafts=None) -> list[Row]:
        """One :class:`Row` per input: ``audio[j]`` the list of its segments' embeddings, ``langs[j]`` its language
        embedding row (None: 0), ``drafts[j]`` its CTC frame argmaxes (None: no draft)."""
        n = len(audio)
        langs = [None] * n if langs is None else list(langs)
        drafts = [None] * n if drafts is None else list(drafts)
        if len(langs) != n or len(drafts) != n:
            raise ValueError("audio, langs and drafts: one entry per input")
        out = []
        for j in range(n):
            if not audio[j]:
                raise ValueError(f"input {j}: no segment")
            segments = [s.to(self.device, self.layout.dtype) for s in audio[j]]
            out.append(Row(index=j, segments=len(segments), lang=int(langs[j] or 0), audio=segments,
                           frames=as_frames(drafts[j])))
        return out

    def context(self, row: Row, i: int) -> Tensor:
        """Decoder input embeddings ``[C, D]`` of segment ``i`` of ``row``, ending with <bos>."""
        return self.layout(row, i)

    def result(self, row: Row):
        ids = [t for segment in row.tokens for t in segment if t not in (PAD, BOS, EOS)]
        return ids if self.tokenizer is None else self.tokenizer.decode(ids)

    # ------------------------------------------------------------------ decoding

    def decoder(self, beams: int, length_norm: bool):
        """The decoder of this search (see :func:`search_key`); the pool releases the others' caches."""
        dec = self.pool.take(search_key(beams, length_norm, self.draft_tokens))
        dec.phase = self.timed
        self.last_decoder = dec
        return dec

    def transcribe_rows(self, rows: list[Row], beams: int = 1, length_norm: bool = False) -> list:
        """Decode every segment of every row as one stream per row; the rows share the decoder's slots, and the
        drafted decoder takes each segment's draft from the row's CTC frames as the segment is admitted."""
        dec = self.decoder(beams, length_norm)
        streams = SegmentStreams(rows, self.layout, self.timed)
        drafted = isinstance(dec, SpecDecoder)
        if drafted:
            dec.drafts = streams.draft
        try:
            with self.timed("decoder"):
                dec.decode_streams(len(rows), streams.first, streams.advance)
        finally:
            if drafted:
                dec.drafts = lambda j: None  # the rows (their embeddings) are not held after the call
        return [self.result(r) for r in rows]

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
        drafted = search_key(beams, length_norm, self.draft_tokens)[0] == "spec"
        if not drafted:
            drafts = None  # only the drafted search reads frames
        elif drafts is None and self.drafter is not None:
            with self.timed("drafter"):
                drafts = self.drafter.frame_ids(audio)
        return self.transcribe_rows(self.rows(audio, langs, drafts), beams, length_norm)


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


__all__ = ["DecoderPool", "PromptLayout", "SegmentStreams", "Transcriber", "frames_from_tokens", "search_key"]

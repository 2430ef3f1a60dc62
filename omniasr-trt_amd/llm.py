"""Streaming constants and host-side rules of the omniASR LLM greedy search, plus the CTC-draft rows.

The rules kept from the reference (src/omniasr_trt/llm.py:1-59): greedy on the log-softmax, stop at EOS, at
position ``MAX_GEN - 4``, or when the 100 tokens before a position that is a multiple of 250 compress more than
4x under zlib (checked only past context + 100).  Each 15 s segment is decoded with the previous segment's audio
and text as its context; a CTC drafter's frame argmaxes give each segment a draft text
(:meth:`Row.draft`, src/omniasr_trt/llm.py:74-85).
"""

from __future__ import annotations

import zlib
from dataclasses import dataclass, field

import numpy as np
from torch import Tensor

from .modeling import HOP

SEGMENT = 15 * 16000
# A segment's draft also takes this many CTC frames from before and after its own span, so that a word cut by the
# segment boundary is still drafted whole.
DRAFT_MARGIN = (25, 50)
BOS, PAD, EOS = 0, 1, 2
MAX_GEN = 8192
CHECK_EVERY, CHECK_WINDOW, CHECK_RATIO = 250, 100, 4.0


def compression_ratio(tokens: np.ndarray) -> float:
    """The repetition test: length of ``np.array_str`` of the int32 ids (newlines removed) over its zlib size
    (src/omniasr_trt/llm.py:44-47)."""
    data = np.array_str(np.asarray(tokens).astype(np.int32)).replace("\n", "").encode("utf-8")
    return len(data) / len(zlib.compress(data))


def early_stop_index(out: np.ndarray, start: int, stop: int, ctx: int) -> int | None:
    """First checked position t in [start, stop] (a multiple of ``CHECK_EVERY``, t > ctx + ``CHECK_WINDOW``) whose
    preceding ``CHECK_WINDOW`` tokens compress more than ``CHECK_RATIO``; ``out[t]`` (the token predicted from input
    position t) is kept and the row ends after it (src/omniasr_trt/llm.py:50-59)."""
    t = -(-start // CHECK_EVERY) * CHECK_EVERY
    while t <= stop:
        if t > ctx + CHECK_WINDOW and compression_ratio(out[t - CHECK_WINDOW: t]) > CHECK_RATIO:
            return t
        t += CHECK_EVERY
    return None


def frames_to_draft(frames: np.ndarray, segment: int, segment_samples: int = SEGMENT) -> tuple[list[int], int]:
    """Segment ``segment``'s draft from per-20 ms CTC argmaxes ``frames``: the frames of the segment and a margin of
    ``DRAFT_MARGIN`` frames around it, repeats collapsed, blank / pad / EOS (ids <= 2) dropped; and the draft position
    where the segment's own frames start (src/omniasr_trt/llm.py:74-85)."""
    lo, hi = segment * segment_samples // HOP, (segment + 1) * segment_samples // HOP
    begin = max(0, lo - DRAFT_MARGIN[0])
    ids = np.asarray(frames, dtype=np.int64)[begin: hi + DRAFT_MARGIN[1]]
    keep = np.ones(len(ids), dtype=bool)
    keep[1:] = ids[1:] != ids[:-1]
    keep &= ids > EOS
    before = int(keep[: lo - begin].sum())
    return ids[keep].tolist(), before


@dataclass
class Row:
    """One input's streaming state: its segments' decoder embeddings and tokens, and its CTC frames."""

    index: int
    segments: int
    lang: int = 0
    audio: list = field(default_factory=list)  # per segment: [F, D] decoder embeddings of its audio frames
    tokens: list = field(default_factory=list)  # the decoded ids of each segment so far, one list per segment
    frames: np.ndarray | None = None  # draft source: CTC argmax of each 20 ms frame

    def draft(self, i: int) -> tuple[list[int], int] | None:
        """Segment i's draft and the draft position where its own frames start; None without frames."""
        if self.frames is None:
            return None
        return frames_to_draft(self.frames, i, SEGMENT)  # the module's SEGMENT at call time


def as_frames(d) -> np.ndarray | None:
    if d is None:
        return None
    return np.asarray(d.cpu() if isinstance(d, Tensor) else d, dtype=np.int64)


__all__ = ["BOS", "CHECK_EVERY", "CHECK_RATIO", "CHECK_WINDOW", "DRAFT_MARGIN", "EOS", "HOP", "MAX_GEN", "PAD",
           "Row", "SEGMENT", "as_frames", "compression_ratio", "early_stop_index", "frames_to_draft"]

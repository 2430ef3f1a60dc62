"""The transcriber's decoding side on the HIP kernels against the reference-order loop (src tests/test_spec.py:163-184):
multi-segment inputs whose segment i + 1 is decoded with segment i's audio and tokens as context, CTC frame drafts
turned into each segment's draft by ``Row.draft`` and handed to the drafted decoder as the segment is admitted
(frames -> ``Row.draft`` -> ``SpecDecoder.drafts`` -> ``filled`` -> ``propose``), and the choice of decoder.

The oracle side restates the context layout (src/omniasr_trt/llm.py:160-173) on fp64 copies of the same weights and
decodes each segment with ``oracle.reference.greedy_reference`` in the reference's order."""

import sys

import numpy as np
import pytest
import torch

from oracle import reference as oref
from omniasr_trt_amd import llm
from omniasr_trt_amd.beam import BeamDecoder
from omniasr_trt_amd.decode import GreedyDecoder
from omniasr_trt_amd.modeling import HOP
from omniasr_trt_amd.spec import SpecDecoder
from omniasr_trt_amd.transcribe import Transcriber, frames_from_tokens

from test_beam_gpu import ROBUST
from test_decode_gpu import gpu_pair

pytestmark = pytest.mark.gpu

FRAMES = 100  # CTC frames per segment in these tests (the segment length is patched to 100 * HOP samples)
VOCAB = 12
SHAPES = [(17, 30, 9), (25,), (12, 40), (33, 8, 21, 14), (19,)]  # CTC frames of each input's segments


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def oracle_context(sd, vocab, lang, audio, tokens, i):
    """Segment i's context in fp64, restated: [lang] <lid> (audio_{i-1} <regular> <bos> text_{i-1} <eos>) audio_i
    <last|regular> <bos>."""
    text = sd["text_frontend.weight"]
    lid, last_seg, regular = vocab, vocab + 1, vocab + 2
    parts = [sd["lang_embeddings.weight"][lang: lang + 1], text[[lid]]]
    if i > 0:
        parts += [audio[i - 1].double(), text[[regular, llm.BOS, *tokens[i - 1], llm.EOS]]]
    parts += [audio[i].double(), text[[last_seg if i == len(audio) - 1 else regular, llm.BOS]]]
    return torch.cat(parts)


def oracle_transcripts(ref_dec, inputs, langs):
    """Per input the per-segment greedy tokens, each segment decoded after the previous one (its context)."""
    out = []
    for audio, lang in zip(inputs, langs):
        tokens = []
        for i in range(len(audio)):
            margins = []
            tokens.append(oref.greedy_reference(ref_dec, oracle_context(ref_dec.sd, VOCAB, lang, audio, tokens, i),
                                                margins=margins))
            assert min(margins) > 1e-3  # fp32 and fp64 agree far from ties
        out.append(tokens)
    return out


@pytest.fixture(scope="module")
def case(cuda):
    m, ref_dec = gpu_pair(24)
    g = torch.Generator().manual_seed(77)
    inputs = [[torch.randn(f, 32, generator=g) for f in segs] for segs in SHAPES]
    langs = [1, None, 3, 0, 4]
    ref = oracle_transcripts(ref_dec, inputs, [0 if x is None else x for x in langs])
    say(f"oracle tokens per segment: {[[len(t) for t in r] for r in ref]}")
    assert sum(len(t) for r in ref for t in r) >= 60
    return m, inputs, langs, ref


def flat(per_segment):
    return [t for seg in per_segment for t in seg]


class FakeDrafter:
    """A CTC drafter stand-in: ``frame_ids`` returns fixed frame argmaxes per input."""

    def __init__(self, frames):
        self.frames = frames
        self.calls = 0

    def frame_ids(self, audio):
        self.calls += 1
        assert len(audio) == len(self.frames)
        return self.frames


def test_frame_drafts_through_the_transcriber(case, monkeypatch):
    m, inputs, langs, ref = case
    monkeypatch.setattr(llm, "SEGMENT", FRAMES * HOP)
    want = [flat(r) for r in ref]
    rng = np.random.default_rng(0)
    clean = [frames_from_tokens(r, FRAMES, rng) for r in ref]
    noisy = [frames_from_tokens(r, FRAMES, rng, substitute=0.1, vocab=VOCAB) for r in ref]
    t = Transcriber(m, max_batch=3, draft_tokens=4, reserve=16)
    say("transcriber: clean frame drafts")
    assert t.transcribe(inputs, langs, drafts=clean) == want
    dec = t.last_decoder
    assert isinstance(dec, SpecDecoder)
    per_step = dec.stats["tokens"] / dec.stats["rows_steps"]
    say(f"transcriber: {per_step:.2f} tokens per row-step with clean drafts")
    assert per_step > 1.5
    say("transcriber: CTC-like drafts (10% substitutions), some inputs without frames")
    assert t.transcribe(inputs, langs, mode="fast", drafts=noisy) == want  # the reference's keyword and default
    with pytest.raises(ValueError, match="reference"):
        t.transcribe(inputs, langs, mode="reference")  # the reference's batch-1 loops are not part of this package
    assert t.transcribe(inputs, langs, drafts=[None, noisy[1], None, clean[3], None]) == want
    say("transcriber: a drafter object, then own tokens only")
    t.drafter = FakeDrafter(noisy)
    assert t.transcribe(inputs, langs) == want and t.drafter.calls == 1
    t.drafter = None
    assert t.transcribe(inputs, langs) == want
    assert dec.drafts(0) is None  # the rows are not held after a call


def test_decoder_choice(case, monkeypatch):
    m, inputs, langs, ref = case
    monkeypatch.setattr(llm, "SEGMENT", FRAMES * HOP)
    want = [flat(r) for r in ref]
    t = Transcriber(m, max_batch=3, draft_tokens=4, reserve=16)
    assert t.transcribe(inputs, langs) == want
    spec_dec = t.last_decoder
    t.draft_tokens = 0  # one token per step
    assert t.transcribe(inputs, langs) == want
    assert isinstance(t.last_decoder, GreedyDecoder) and not isinstance(t.last_decoder, SpecDecoder)
    assert spec_dec.capacity == 0  # released when another decoder took over
    say("transcriber: beam search with 3 beams (segment by segment, against the decoder run directly)")
    got = t.transcribe(inputs, langs, beams=3)
    assert isinstance(t.last_decoder, BeamDecoder) and t.last_decoder.beams == 3
    assert t.pool.decoders[("greedy",)].capacity == 0
    # the same search run by hand: each input's segments in order, contexts from the beam tokens
    direct = BeamDecoder(m, beams=3, max_batch=3, reserve=16)
    for j, audio in enumerate(inputs):
        row = llm.Row(index=j, segments=len(audio), lang=0 if langs[j] is None else langs[j],
                      audio=[a.cuda() for a in audio])
        for i in range(len(audio)):
            row.tokens.append(direct.generate([t.context(row, i)])[0])
        assert got[j] == flat(row.tokens), j


def oracle_beam_transcripts(ref_dec, inputs, langs, beams, length_norm):
    """Per input the per-segment beam-search tokens, each segment's context built from the previous segment's."""
    out = []
    for audio, lang in zip(inputs, langs):
        tokens = []
        for i in range(len(audio)):
            margins = []
            ctx = oracle_context(ref_dec.sd, VOCAB, lang, audio, tokens, i)
            tokens.append(oref.beam_reference(ref_dec, ctx, beams, length_norm, margins=margins))
            assert min(margins) > ROBUST, f"segment {i} has a near-tie ({min(margins):.1e})"
        out.append(tokens)
    return out


@pytest.mark.parametrize("beams,length_norm,seed", [(3, False, 77), (3, True, 89)])
def test_beam_transcripts_vs_oracle(case, monkeypatch, beams, length_norm, seed):
    """Beam transcription end to end (src tests/test_beam.py:45-62): every input's segments in order, segment i + 1's
    context holding segment i's beam tokens, fewer groups than inputs (a finished group takes the next segment or
    the next input), against the oracle's beam search of each segment's context in the reference's order.  The
    inputs of each seed are chosen free of near-ties in the oracle's choices."""
    m, _, langs, _ = case
    monkeypatch.setattr(llm, "SEGMENT", FRAMES * HOP)
    g = torch.Generator().manual_seed(seed)
    inputs = [[torch.randn(f, 32, generator=g) for f in segs] for segs in SHAPES]
    ref_dec = oref.Fp64Decoder(m)  # the case's own fp32 weights
    want = [flat(r) for r in oracle_beam_transcripts(ref_dec, inputs, [0 if x is None else x for x in langs], beams,
                                                     length_norm)]
    say(f"transcriber: beams={beams} length_norm={length_norm}, {sum(map(len, want))} oracle tokens")
    t = Transcriber(m, max_batch=2, reserve=16, beams=beams, length_norm=length_norm)
    assert t.transcribe(inputs, langs) == want
    assert isinstance(t.last_decoder, BeamDecoder) and t.last_decoder.beams == beams
    # the same search asked for per call from a greedy transcriber
    g = Transcriber(m, max_batch=2, reserve=16, draft_tokens=0)
    assert g.transcribe(inputs, langs, beams=beams, length_norm=length_norm) == want

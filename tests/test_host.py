"""Host-side logic that needs no GPU: the reference's launch-split rule, module names of the decoder, constants."""

import numpy as np
import pytest
import torch

from omniasr_trt_amd import decode, kernels, llm, modeling, spec


def test_splits_for_is_the_reference_rule():
    # src/omniasr_trt/kernels.py:393-400: a power of two, about ``programs`` programs, 2 * block keys per split at least
    assert kernels.splits_for(8, 32, 2560, 32, 264) == (1, 2560)
    assert kernels.splits_for(8, 8, 2048, 64, 264) == (4, 512)
    assert kernels.splits_for(1, 8, 256, 64, 264) == (4, 64)  # 264 // 8 = 33 wanted; 4 * 64 keys fill 256
    assert kernels.splits_for(4, 8, 700, 32, 264) == (8, 96)


def test_next_power_of_2():
    assert [kernels.next_power_of_2(n) for n in (0, 1, 2, 3, 225, 256, 257)] == [1, 1, 2, 4, 256, 256, 512]


def test_decoder_parameter_names_are_fairseq2s():
    cfg = modeling.DecoderConfig(model_dim=32, num_layers=2, num_heads=2, ffn_dim=24, vocab_size=12, num_langs=5)
    names = set(modeling.DecoderModel(cfg).state_dict())
    want = {"text_frontend.weight", "final_proj.weight", "lang_embeddings.weight", "llama_decoder.layer_norm.weight"}
    for i in range(2):
        p = f"llama_decoder.layers.{i}."
        want |= {p + "self_attn_layer_norm.weight", p + "ffn_layer_norm.weight"}
        want |= {p + f"self_attn.{x}_proj.weight" for x in ("q", "k", "v", "output")}
        want |= {p + f"ffn.{x}_proj.weight" for x in ("gate", "inner", "output")}
    assert names == want


def test_rope_table_follows_the_model_device_and_stays_fp32():
    cfg = modeling.DecoderConfig(model_dim=32, num_layers=1, num_heads=2, ffn_dim=24, vocab_size=12, num_langs=5)
    m = modeling.DecoderModel(cfg).to(torch.bfloat16)
    assert m.rope.dtype == torch.float32 and m.rope.shape == (8192, 8, 2)
    assert m.double().rope.dtype == torch.float32


def test_reference_constants():
    assert (spec.NGRAM, spec.BEHIND, spec.AHEAD, spec.SELF_WINDOW, spec.SELF_MIN) == (8, 64, 160, 256, 3)
    assert spec.REACH == ((1, 1), (4, 2), (12, 4), (40, 6)) and spec.DRAFT_CAPACITY == 1024
    assert decode.LIMIT == 8188 and decode.KEY_BUCKET == 256 and decode.CONTEXT_FLOOR == 2048
    assert (llm.BOS, llm.PAD, llm.EOS) == (0, 1, 2)


def test_row_draft():
    frames = np.array([0, 0, 5, 5, 6, 0, 6, 7, 2, 7] * 100)
    r = llm.Row(index=0, segments=2, frames=frames)
    ids, before = r.draft(0)
    assert before == 0 and ids[:6] == [5, 6, 6, 7, 7, 5]
    assert llm.Row(index=1, segments=1).draft(0) is None


def test_decoders_refuse_a_cpu_model():
    cfg = modeling.DecoderConfig(model_dim=32, num_layers=1, num_heads=2, ffn_dim=24, vocab_size=12, num_langs=5)
    with pytest.raises(RuntimeError):
        decode.GreedyDecoder(modeling.DecoderModel(cfg))
    with pytest.raises(ValueError):
        decode.GreedyDecoder(modeling.DecoderModel(cfg), fused=False)


def test_bench_runs_one_gpu_only():
    """bench.py measures one GPU: any other --gpus exits with status 2 and says why, before touching a device."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "8"], capture_output=True, text=True,
                       timeout=120, cwd=root)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_synthetic_frames_give_back_each_segments_tokens(monkeypatch):
    """transcribe.frames_from_tokens (the CTC stand-in of the tests and the benchmark): Row.draft of segment i
    returns the tokens of the neighbouring frames' margin and then segment i's own, starting at ``before``."""
    from omniasr_trt_amd.transcribe import frames_from_tokens

    monkeypatch.setattr(llm, "SEGMENT", 100 * modeling.HOP)
    rng = np.random.default_rng(4)
    segments = [[int(x) for x in rng.integers(3, 50, n)] for n in (20, 7, 33, 0, 12)]
    frames = frames_from_tokens(segments, 100, rng)
    assert len(frames) == 500
    row = llm.Row(index=0, segments=5, frames=frames)
    for i, seg in enumerate(segments):
        ids, before = row.draft(i)
        assert ids[before: before + len(seg)] == seg, i
    noisy = frames_from_tokens(segments, 100, np.random.default_rng(4), substitute=0.5, vocab=50)
    ids, before = llm.Row(index=0, segments=5, frames=noisy).draft(2)
    assert ids[before: before + 33] != segments[2] and len(ids[before: before + 33]) == 33


def test_prompt_layout_and_search_choice():
    """The transcriber's segment prompt (src/omniasr_trt/llm.py:160-173): [lang] <lid> (audio_{i-1} <regular> <bos>
    text_{i-1} <eos>) audio_i <last|regular> <bos>, with the three markers after the text vocabulary; and the decoder
    each search runs on (llm.py:284-313)."""
    from omniasr_trt_amd import transcribe

    cfg = modeling.DecoderConfig(model_dim=16, num_layers=1, num_heads=2, ffn_dim=24, vocab_size=12, num_langs=5)
    m = modeling.DecoderModel(cfg)
    t = transcribe.Transcriber(m)
    g = torch.Generator().manual_seed(3)
    (row,) = t.rows([[torch.randn(4, 16, generator=g), torch.randn(2, 16, generator=g), torch.randn(3, 16, generator=g)]],
                    langs=[3])
    row.tokens += [[5, 6], [7]]
    lid, last, regular = 12, 13, 14
    assert t.layout.parts(row, 0)[1] == ("ids", [lid]) and t.layout.parts(row, 0)[-1] == ("ids", [regular, llm.BOS])
    assert t.layout.parts(row, 2)[-1] == ("ids", [last, llm.BOS])  # the input's last segment
    assert t.layout.parts(row, 1)[3] == ("ids", [regular, llm.BOS, 5, 6, llm.EOS])
    text, langs = m.text_frontend.weight, m.lang_embeddings.weight
    for i in range(3):
        want = [langs[3:4], text[[lid]]]
        if i:
            want += [row.audio[i - 1], text[[regular, llm.BOS, *row.tokens[i - 1], llm.EOS]]]
        want += [row.audio[i], text[[last if i == 2 else regular, llm.BOS]]]
        assert torch.equal(t.context(row, i), torch.cat(want)), i
    assert transcribe.search_key(1, False, 4) == ("spec", 4)
    assert transcribe.search_key(1, False, 0) == ("greedy",)
    assert transcribe.search_key(5, False, 4) == ("beam", 5, False)
    assert transcribe.search_key(1, True, 4) == ("beam", 1, True)  # length normalisation is a beam search
    with pytest.raises(ValueError):
        t.rows([[torch.zeros(1, 16)]], langs=[0, 1])

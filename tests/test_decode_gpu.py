"""The decoders on the HIP kernels against the reference-order greedy loop (oracle, fp64 on the CPU), on a small
random fp32 model: speculative decoding gives exactly the greedy tokens whatever the drafts
(src tests/test_spec.py:111-198, tests/test_kernels.py:58-95)."""

import copy
import sys

import numpy as np
import pytest
import torch

from oracle import reference as oref
from omniasr_trt_amd import decode, llm, spec
from omniasr_trt_amd.decode import GreedyDecoder
from omniasr_trt_amd.modeling import DecoderConfig, DecoderModel
from omniasr_trt_amd.spec import SpecDecoder

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def small_model(seed: int, vocab: int = 12) -> DecoderModel:
    """d 32, 2 layers, 2 heads (head_dim 16), ffn 24; weights N(0, 0.5), LM head x4 (peaked distributions)."""
    torch.manual_seed(seed)
    cfg = DecoderConfig(model_dim=32, num_layers=2, num_heads=2, ffn_dim=24, vocab_size=vocab, num_langs=5)
    m = DecoderModel(cfg).double().eval()
    with torch.no_grad():
        for p in m.parameters():
            p.normal_(0, 0.5)
        m.final_proj.weight.mul_(4)
    return m


def gpu_pair(seed: int, edit=None):
    """The fp32 GPU model and the oracle built from the very same fp32 weights."""
    m = small_model(seed)
    if edit is not None:
        edit(m)
    g = copy.deepcopy(m).float().cuda()
    return g, oref.Fp64Decoder(g)


def contexts(seed, lengths):
    torch.manual_seed(seed)
    return [torch.randn(n, 32).float() for n in lengths]


def noisy(tokens, rng, vocab=12):
    """A draft with tokens changed, dropped and added, and a tail of junk (src tests/test_spec.py:27-40)."""
    out = []
    for t in tokens:
        r = rng.random()
        if r < 0.1:
            out.append(int(rng.integers(3, vocab)))
        elif r < 0.15:
            continue
        elif r < 0.2:
            out += [t, int(rng.integers(3, vocab))]
        else:
            out.append(t)
    return out + [int(x) for x in rng.integers(3, vocab, 5)]


def run(dec, ctxs, drafts):
    dec.drafts = lambda j: drafts[j]
    return dec.generate([c.cuda() for c in ctxs])


def test_greedy_decoder_matches_reference_order(cuda):
    m, ref_dec = gpu_pair(2)
    ctxs = contexts(3, (5, 33, 17, 60))
    ref = [oref.greedy_reference(ref_dec, c) for c in ctxs]
    say("greedy decoder, graphs")
    got = GreedyDecoder(m, max_batch=4, sync_every=8, reserve=64).generate([c.cuda() for c in ctxs])
    assert got == ref
    say("greedy decoder, eager")
    assert GreedyDecoder(m, max_batch=4, sync_every=8, reserve=64, graphs=False).generate([c.cuda() for c in ctxs]) \
        == ref


def test_streams_across_calls(cuda):
    """Continuous batching: refills of scattered slots, more streams than slots, then smaller calls."""
    m, ref_dec = gpu_pair(7)
    dec = GreedyDecoder(m, max_batch=3, sync_every=4, reserve=8)
    for n, lengths in ((7, (250, 40, 5, 251, 90, 12, 248)), (2, (30, 8)), (5, (60, 252, 9, 33, 100)), (1, (17,))):
        ctxs = contexts(8 + n, lengths[:n])
        say(f"streams: {n} contexts")
        assert dec.generate([c.cuda() for c in ctxs]) == [oref.greedy_reference(ref_dec, c) for c in ctxs], lengths


@pytest.mark.parametrize("draft_tokens", [1, 4, 8])
def test_same_tokens_as_greedy(cuda, draft_tokens):
    m, ref_dec = gpu_pair(24)  # seed 24: every context yields 7-44 greedy tokens
    ctxs = contexts(22, (40, 7, 251, 90, 13, 60))
    ref = [oref.greedy_reference(ref_dec, c) for c in ctxs]
    assert min(len(r) for r in ref) >= 3
    rng = np.random.default_rng(0)
    dec = SpecDecoder(m, draft_tokens=draft_tokens, max_batch=4, sync_every=3, reserve=8)
    say(f"spec k={draft_tokens}: perfect drafts")
    assert run(dec, ctxs, [(r + [5, 6, 7], 0) for r in ref]) == ref  # drafts that continue beyond the reference's EOS
    tokens_per_step = dec.stats["tokens"] / dec.stats["rows_steps"]
    say(f"spec k={draft_tokens}: noisy drafts ({tokens_per_step:.2f} tokens/row-step with perfect ones)")
    assert run(dec, ctxs, [(noisy(r, rng), 0) for r in ref]) == ref
    assert run(dec, ctxs, [(noisy(r[3:], rng), 2) for r in ref]) == ref  # starting mid-draft
    assert run(dec, ctxs, [None, ([], 0), *[(list(rng.integers(3, 12, 30)), 0) for _ in ctxs[2:]]]) == ref
    if draft_tokens > 1:  # exact drafts are accepted, so a row gains more than one token a step
        assert tokens_per_step > 1.5


def test_length_limit_and_eos_inside_a_step(cuda, monkeypatch):
    m, ref_dec = gpu_pair(23, edit=lambda m: m.final_proj.weight.data[llm.EOS].mul_(0.3))  # long generations
    monkeypatch.setattr(decode, "LIMIT", 70)
    monkeypatch.setattr(spec, "LIMIT", 70)
    ctxs = contexts(24, (5, 30, 64, 69, 12))
    ref = [oref.greedy_reference(ref_dec, c, limit=70) for c in ctxs]
    say("limit 70: greedy")
    assert GreedyDecoder(m, max_batch=3, sync_every=4, reserve=8).generate([c.cuda() for c in ctxs]) == ref
    say("limit 70: drafted")
    dec = SpecDecoder(m, draft_tokens=6, max_batch=3, sync_every=4, reserve=8)
    assert run(dec, ctxs, [(r + [4] * 20, 0) for r in ref]) == ref


def test_repetition_stop_and_cache_growth(cuda):
    m, ref_dec = gpu_pair(15, edit=lambda m: m.final_proj.weight.data[llm.EOS].zero_())  # no EOS
    ctxs = contexts(25, (5, 60, 140, 151))
    ref = [oref.greedy_reference(ref_dec, c) for c in ctxs]
    rng = np.random.default_rng(3)
    dec = SpecDecoder(m, draft_tokens=4, max_batch=3, sync_every=5, reserve=8)
    dec.context_floor = 0
    say("repetition stop, growing caches")
    assert run(dec, ctxs, [(noisy(r, rng), 0) for r in ref]) == ref
    assert dec.stats["grows"] >= 1


def test_own_tokens_without_draft(cuda):
    """No draft: a repetition loop is proposed from the row's own tokens (several tokens per step)."""
    m, ref_dec = gpu_pair(15, edit=lambda m: m.final_proj.weight.data[llm.EOS].zero_())
    ctxs = contexts(26, (5, 60, 99))
    ref = [oref.greedy_reference(ref_dec, c) for c in ctxs]
    dec = SpecDecoder(m, draft_tokens=4, max_batch=3, sync_every=5, reserve=8)
    assert run(dec, ctxs, [None] * len(ctxs)) == ref
    assert dec.stats["tokens"] / dec.stats["rows_steps"] > 1.5


def test_graph_replays_equal_eager_steps(cuda):
    m, _ = gpu_pair(24)
    ctxs = contexts(22, (40, 7, 251, 90, 13, 60))
    drafts = [(list(range(3, 12)) * 3, 0)] * len(ctxs)
    a = SpecDecoder(m, draft_tokens=4, max_batch=4, sync_every=3, reserve=8, graphs=True)
    b = SpecDecoder(m, draft_tokens=4, max_batch=4, sync_every=3, reserve=8, graphs=False)
    assert run(a, ctxs, drafts) == run(b, ctxs, drafts)
    assert a.stats["rows_steps"] == b.stats["rows_steps"] and a.stats["captures"] > 0


@pytest.mark.parametrize("model_dim,heads", [(256, 2), (512, 1)])
def test_bf16_prefill_kernel_matches_torch_attention(cuda, monkeypatch, model_dim, heads):
    """A bf16 model with head dim 128 (the causal kernel) or 512 (the slice-per-wave kernel): the prefill through
    kernels.prefill_attention gives the log-probabilities of the fp32 torch attention path within bf16 tolerance,
    for contexts of different lengths in permuted cache rows."""
    torch.manual_seed(31)
    cfg = DecoderConfig(model_dim=model_dim, num_layers=2, num_heads=heads, ffn_dim=64, vocab_size=40, num_langs=5)
    m = DecoderModel(cfg).eval()
    with torch.no_grad():
        for p in m.parameters():
            p.normal_(0, 0.05)
    m = m.to(torch.bfloat16).cuda()
    dec = GreedyDecoder(m, max_batch=3, graphs=False, reserve=8)
    ctxs = [torch.randn(n, model_dim).to(torch.bfloat16).cuda() for n in (70, 5, 133)]

    def prefill():
        k = torch.zeros(2, 4, heads, 160, model_dim // heads, dtype=torch.bfloat16, device=cuda)
        v = torch.zeros_like(k)
        logp = dec.prefill_into(ctxs, [3, 0, 2], k, v)
        torch.cuda.synchronize()
        return logp.float().cpu(), k.cpu(), v.cpu()

    fused = prefill()
    monkeypatch.setattr(decode.kernels, "prefill_supported", lambda dtype, head_dim: False)
    plain = prefill()
    torch.testing.assert_close(fused[1][0], plain[1][0], atol=0, rtol=0)  # layer 0: the same RoPE writes
    torch.testing.assert_close(fused[0], plain[0], atol=5e-2, rtol=5e-2)


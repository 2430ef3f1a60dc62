"""Pins ``oracle.step.NumpySpecDecoder`` -- the whole drafted step in numpy, timed as the benchmark's CPU baseline --
against the fp64 reference-order loop (CPU): on a small fp32 model, drafted decoding with perfect, noisy and no
drafts gives exactly ``oracle.reference.greedy_reference``'s tokens, and the verify logits of every step agree with
an fp64 forward of the decoder over the same token sequence to fp32 precision."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import reference as oref
from oracle import step as ostep
from omniasr_trt_amd import spec

from test_decode_gpu import contexts, noisy, small_model

EOS, PAD, LIMIT = 2, 1, 8188
CAP = 512


def prefilled(ref_dec, ctxs, k_drafts, drafts):
    """Caches and slot state after the prefill of ``ctxs`` (fp64 forward, K/V stored in fp32), drafts loaded."""
    cfg = ref_dec.cfg
    layers, heads, dim = cfg.num_layers, cfg.num_heads, cfg.model_dim // cfg.num_heads
    b = len(ctxs)
    kc = np.zeros((layers, b, heads, CAP, dim), dtype=np.float32)
    vc = np.zeros_like(kc)
    st = {"tok": np.zeros(b, np.int64), "last": np.zeros(b, np.int64), "done": np.zeros(b, bool),
          "out": np.full((b, CAP), PAD, np.int32), "draft": np.full((b, spec.DRAFT_CAPACITY), -1, np.int32),
          "draft_len": np.zeros(b, np.int64), "next": np.zeros(b, np.int64), "first": np.zeros(b, np.int64),
          "start": np.zeros(b, np.int64)}
    for s, ctx in enumerate(ctxs):
        c = ctx.size(0)
        cache = [None] * layers
        h = ref_dec.forward(ctx.double(), torch.arange(c), cache)
        first = int(F.log_softmax(ref_dec.logits(h[-1]), -1).argmax())
        for i in range(layers):
            kc[i, s, :, :c] = cache[i][0].permute(1, 0, 2).float().numpy()
            vc[i, s, :, :c] = cache[i][1].permute(1, 0, 2).float().numpy()
        st["out"][s, c - 1] = first
        st["tok"][s], st["last"][s], st["first"][s] = first, c - 1, c - 1
        st["done"][s] = first == EOS
        ids, where = drafts[s] if drafts[s] is not None else ([], 0)
        st["draft"][s, : len(ids)] = ids
        st["draft_len"][s], st["next"][s] = len(ids), where + 1
    w = ostep.weights_from_state_dict({k: v.float() for k, v in ref_dec.sd.items()})
    npdec = ostep.NumpySpecDecoder(w, layers, heads, cfg.rms_eps, oref.rope_table(dim, cfg.max_seq_len).numpy(), kc,
                                   vc, st, k_drafts, spec.NGRAM, spec.BEHIND, spec.AHEAD, spec.REACH,
                                   spec.SELF_WINDOW, spec.SELF_MIN, LIMIT, EOS)
    return npdec, st


def fp64_logits(ref_dec, ctx, generated, fed):
    """fp64 logits at the positions of ``fed`` after the context and the tokens generated so far."""
    emb = ref_dec.sd["text_frontend.weight"]
    seq = torch.cat([ctx.double(), emb[torch.tensor(generated + fed, dtype=torch.long)]])
    h = ref_dec.forward(seq, torch.arange(seq.size(0)), [None] * ref_dec.layers)
    return ref_dec.logits(h[-len(fed):]).numpy()


@pytest.mark.parametrize("k,kind", [(4, "perfect"), (4, "noisy"), (2, "none"), (6, "noisy")])
def test_numpy_drafted_step_is_the_greedy_search(k, kind):
    m = small_model(24).float()
    ref_dec = oref.Fp64Decoder(m)
    ctxs = contexts(22, (40, 7, 90))
    ref = [oref.greedy_reference(ref_dec, c) for c in ctxs]
    rng = np.random.default_rng(k)
    drafts = {"perfect": [(r + [5, 6, 7], 0) for r in ref], "noisy": [(noisy(r, rng), 0) for r in ref],
              "none": [None] * len(ref)}[kind]
    npdec, st = prefilled(ref_dec, ctxs, k, drafts)
    start_pos = st["last"].copy()
    steps = accepted = 0
    while not st["done"].all():
        before_last, before_done = st["last"].copy(), st["done"].copy()
        keys = min(CAP, -(-(int(st["last"].max()) + 8 * (k + 1) + 2) // 256) * 256)
        accepted += npdec.step(keys)
        steps += 1
        logits = npdec.last_logits.reshape(len(ctxs), k + 1, -1)
        for s in np.flatnonzero(~before_done):
            c = ctxs[s].size(0)
            generated = [int(x) for x in st["out"][s, c - 1: before_last[s]]]  # fed at positions c .. last
            fed = [int(x) for x in npdec.last_tokens[s]]
            want = fp64_logits(ref_dec, ctxs[s], generated, fed)
            scale = float(np.abs(want).max())
            np.testing.assert_allclose(logits[s], want, rtol=1e-4, atol=1e-4 * scale, err_msg=f"step {steps} slot {s}")
        assert steps < 200
    got = [[int(t) for t in st["out"][s, start_pos[s]: st["last"][s] + 1] if t not in (PAD, 0, EOS)]
           for s in range(len(ctxs))]
    assert got == ref
    if kind == "perfect":
        assert accepted / steps > 1.5 * len(ctxs) / 2  # several tokens per step

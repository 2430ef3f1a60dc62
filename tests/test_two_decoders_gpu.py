"""Two drafted decoders stepping on two streams of one GPU at once (a 2-layer bf16 stack, 8 slots x 16 heads x 128:
the verify attention's halves kernel, whose merges take tickets): each decoder's tokens equal its own run alone, bit
for bit, and each decoder's own merge tickets (``GreedyDecoder.attn_tickets``) are distinct and left zero.  (With one
ticket array forced on both, runs on the box also gave equal tokens -- the attention launches, one workgroup per CU,
seldom overlap -- so this checks the decoders under concurrency, not a collision.)"""

import pytest
import torch

import bench
from omniasr_trt_amd import modeling

pytestmark = pytest.mark.gpu

STEPS = 6


def test_two_decoders_on_two_streams(cuda):
    pkg = bench.package()
    cfg = modeling.DecoderConfig(model_dim=2048, num_layers=2, num_heads=16, ffn_dim=2048, vocab_size=1024,
                                 num_langs=4)
    b = bench.SLOTS
    with torch.inference_mode():
        ws = [bench.Workload(pkg, torch, seed=s, cfg=cfg, lo=300, hi=900) for s in (11, 12)]
        assert ws[0].dec.attn_tickets is not ws[1].dec.attn_tickets
        keys = [min(w.dec.capacity, -(-(int(w.lengths.max()) + STEPS * (bench.DRAFT + 1) + 2) // 256) * 256)
                for w in ws]
        alone = []
        for w, k in zip(ws, keys):
            w.restore()
            for _ in range(STEPS):
                w.dec.step(b, k)
            torch.cuda.synchronize()
            alone.append((w.dec.out[:b].clone(), w.dec.last[:b].clone()))
        for w in ws:
            w.restore()
        torch.cuda.synchronize()
        streams = [torch.cuda.Stream(), torch.cuda.Stream()]
        for s in streams:
            s.wait_stream(torch.cuda.current_stream())
        for _ in range(STEPS):  # the two decoders' launches interleaved on their own streams, no synchronisation
            for w, k, s in zip(ws, keys, streams):
                with torch.cuda.stream(s):
                    w.dec.step(b, k)
        torch.cuda.synchronize()
    for i, ((out, last), w) in enumerate(zip(alone, ws)):
        assert torch.equal(w.dec.last[:b], last), i
        assert torch.equal(w.dec.out[:b], out), i
        assert int(w.dec.attn_tickets.abs().sum()) == 0, i
    assert int((alone[0][1] - ws[0].snapshot["last"]).min()) >= STEPS  # every slot advanced every step

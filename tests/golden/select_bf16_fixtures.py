"""Selects the contexts of tests/test_decode_bf16_gpu.py and measures the bf16 error their margin must exceed (CPU).

For a model of that test, candidate contexts N(0, 1) of U[20, 400) positions (context seed 1000 + i, lengths drawn
from numpy's default_rng(5) in order) run through the fp64 reference-order loop (oracle.reference.greedy_reference),
which records the gap between the best and second-best log-probability at every step.  Next to it, a bf16 forward of
the same weights (torch on the CPU: bf16 GEMMs, fp32 RoPE and softmax, bf16 activations) gives the first step's
log-probabilities; the largest difference from fp64 over the eight most likely tokens is the error estimate.  A
candidate is kept when its smallest gap exceeds the margin and it yields at least 3 tokens.

    python tests/golden/select_bf16_fixtures.py d128 100
    python tests/golden/select_bf16_fixtures.py d512 170
"""

from __future__ import annotations

import importlib
import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent
sys.path[:0] = [str(HERE.parents[1]), str(HERE.parent)]
importlib.import_module("omniasr-trt_amd")  # registers the package as omniasr_trt_amd

from oracle import reference as oref  # noqa: E402
from test_decode_bf16_gpu import SHAPES, bf16_model  # noqa: E402


def bf16_first_step(m, ctx: torch.Tensor) -> torch.Tensor:
    """log-softmax after the context's last position, the decoder run in bf16 on the CPU (float32 result)."""
    sd = m.state_dict()
    cfg = m.dec_cfg
    heads, dim = cfg.num_heads, cfg.model_dim // cfg.num_heads
    c = ctx.size(0)
    cs = oref.rope_table(dim, c)[:, None]
    h = ctx.to(torch.bfloat16)
    for i in range(cfg.num_layers):
        p = f"llama_decoder.layers.{i}."
        n = F.rms_norm(h, (h.size(-1),), sd[p + "self_attn_layer_norm.weight"], cfg.rms_eps)
        q, k, v = ((n @ sd[p + f"self_attn.{x}_proj.weight"].t()).view(c, heads, dim) for x in "qkv")
        q, k = oref.apply_rope(q, cs), oref.apply_rope(k, cs)
        o = F.scaled_dot_product_attention(*(t.transpose(0, 1).float() for t in (q, k, v)), is_causal=True)
        h = h + o.to(torch.bfloat16).transpose(0, 1).reshape(c, -1) @ sd[p + "self_attn.output_proj.weight"].t()
        n = F.rms_norm(h, (h.size(-1),), sd[p + "ffn_layer_norm.weight"], cfg.rms_eps)
        gate, inner = n @ sd[p + "ffn.gate_proj.weight"].t(), n @ sd[p + "ffn.inner_proj.weight"].t()
        h = h + (inner * F.silu(gate)) @ sd[p + "ffn.output_proj.weight"].t()
    n = F.rms_norm(h[-1], (h.size(-1),), sd["llama_decoder.layer_norm.weight"], cfg.rms_eps)
    return F.log_softmax(n @ sd["final_proj.weight"].t(), -1).float()


def main(name: str, candidates: int) -> None:
    seed, model_dim, heads, margin, picks = SHAPES[name]
    m = bf16_model(seed, model_dim, heads)
    dec = oref.Fp64Decoder(m)
    rng = np.random.default_rng(5)
    worst, kept = 0.0, []
    for i in range(candidates):
        n = int(rng.integers(20, 400))
        torch.manual_seed(1000 + i)
        ctx = torch.randn(n, model_dim).to(torch.bfloat16)
        gaps: list = []
        tokens = oref.greedy_reference(dec, ctx, margins=gaps)
        cache = [None] * dec.layers
        want = F.log_softmax(dec.logits(dec.forward(ctx.double(), torch.arange(n), cache)[-1]), -1)
        top = want.topk(8).indices
        err = float((bf16_first_step(m, ctx).double()[top] - want[top]).abs().max())
        worst = max(worst, err)
        if min(gaps) > margin and len(tokens) >= 3:
            kept.append((1000 + i, n))
        print(f"candidate {i}: {n} positions, {len(tokens)} tokens, smallest gap {min(gaps):.3f}, bf16 error "
              f"{err:.3f}", flush=True)
    print(f"{name}: largest bf16 error {worst:.3f}; kept (margin {margin}): {kept}; the test uses {picks}")


if __name__ == "__main__":
    main(sys.argv[1], int(sys.argv[2]) if len(sys.argv) > 2 else 100)

"""Reference-order greedy decoding on the CPU in float64 (test infrastructure; see oracle/__init__.py).

Restates ``LLMTranscriber.greedy_reference`` and ``beam_reference`` (src/omniasr_trt/llm.py:182-254) over
``decoder_forward``
(src/omniasr_trt/modeling.py:374-406): prefill all of a context but its final <bos>, then one token at a time,
greedy on the log-softmax, stopping at EOS, at position ``limit``, or at the zlib repetition stop.  Attention is
written out (masked softmax) instead of calling SDPA.  The decoder's weights are read from a model with the
omniASR decoder's parameter names; nothing else of the product is used.
"""

from __future__ import annotations

import math
import zlib

import numpy as np
import torch
import torch.nn.functional as F

BOS, PAD, EOS = 0, 1, 2
MAX_GEN = 8192
CHECK_EVERY, CHECK_WINDOW, CHECK_RATIO = 250, 100, 4.0


def compression_ratio(tokens: np.ndarray) -> float:
    """zlib ratio of ``np.array_str`` of the int32 ids with newlines removed (src/omniasr_trt/llm.py:44-47)."""
    text = np.array_str(np.asarray(tokens).astype(np.int32)).replace("\n", "").encode("utf-8")
    return len(text) / len(zlib.compress(text))


def rope_table(head_dim: int, positions: int, theta: float = 10_000.0) -> torch.Tensor:
    """fp32 [positions, head_dim/2, 2] table as the reference builds it (src/omniasr_trt/modeling.py:293-298)."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    ang = torch.outer(torch.arange(positions, dtype=torch.float32), inv)
    return torch.stack([torch.cos(ang), torch.sin(ang)], -1)


def apply_rope(x: torch.Tensor, cs: torch.Tensor) -> torch.Tensor:
    """Interleaved pairs rotated in fp32, result in x's dtype (src/omniasr_trt/modeling.py:301-306)."""
    xf = x.float().unflatten(-1, (-1, 2))
    re, im = xf[..., 0], xf[..., 1]
    c, s = cs[..., 0], cs[..., 1]
    return torch.stack([re * c - im * s, re * s + im * c], -1).flatten(-2).type_as(x)


def _rms(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


class Fp64Decoder:
    """The decoder's weights in float64 on the CPU and its forward pass with a per-layer K/V cache."""

    def __init__(self, model):
        sd = {k: v.detach().to("cpu", torch.float64) for k, v in model.state_dict().items()}
        cfg = model.dec_cfg
        self.cfg = cfg
        self.heads = cfg.num_heads
        self.eps = cfg.rms_eps
        self.sd = sd
        self.rope = rope_table(cfg.model_dim // cfg.num_heads, cfg.max_seq_len, cfg.rope_theta)
        self.layers = cfg.num_layers

    def embed(self, token: int) -> torch.Tensor:
        return self.sd["text_frontend.weight"][token]

    def forward(self, x: torch.Tensor, positions: torch.Tensor, cache: list) -> torch.Tensor:
        """``x`` [S, D] at ``positions`` [S] after the cached keys; returns the final-norm hidden states [S, D]."""
        sd, h = self.sd, x
        s = x.size(0)
        cs = self.rope[positions][:, None]  # [S, 1, D/2, 2]
        for i in range(self.layers):
            p = f"llama_decoder.layers.{i}."
            n = _rms(h, sd[p + "self_attn_layer_norm.weight"], self.eps)
            q = apply_rope((n @ sd[p + "self_attn.q_proj.weight"].t()).view(s, self.heads, -1), cs)
            k = apply_rope((n @ sd[p + "self_attn.k_proj.weight"].t()).view(s, self.heads, -1), cs)
            v = (n @ sd[p + "self_attn.v_proj.weight"].t()).view(s, self.heads, -1)
            if cache[i] is not None:
                k = torch.cat([cache[i][0], k], 0)
                v = torch.cat([cache[i][1], v], 0)
            cache[i] = (k, v)
            past = k.size(0) - s
            allowed = torch.ones(s, k.size(0), dtype=torch.bool).tril(past)  # causal, aligned to the end
            sc = torch.einsum("shd,lhd->hsl", q, k) * q.size(-1) ** -0.5
            sc = sc.masked_fill(~allowed[None], float("-inf"))
            o = torch.einsum("hsl,lhd->shd", torch.softmax(sc, -1), v).reshape(s, -1)
            h = h + o @ sd[p + "self_attn.output_proj.weight"].t()
            n = _rms(h, sd[p + "ffn_layer_norm.weight"], self.eps)
            gate = n @ sd[p + "ffn.gate_proj.weight"].t()
            inner = n @ sd[p + "ffn.inner_proj.weight"].t()
            h = h + (inner * F.silu(gate)) @ sd[p + "ffn.output_proj.weight"].t()
        return _rms(h, sd["llama_decoder.layer_norm.weight"], self.eps)

    def logits(self, h: torch.Tensor) -> torch.Tensor:
        return h @ self.sd["final_proj.weight"].t()


@torch.inference_mode()
def greedy_reference(dec: Fp64Decoder, ctx: torch.Tensor, limit: int = MAX_GEN - 4,
                     margins: list | None = None) -> list[int]:
    """Greedy tokens of one context [C, D] (ending with <bos>), in the reference's order of computation.

    ``margins``: if a list, receives per step the gap between the largest and the second largest log-probability
    (float64): where it is below the error of another arithmetic (bf16 activations, another summation order), that
    arithmetic may pick the other token, and both are correct roundings of the same search."""
    ctx = ctx.detach().to("cpu", torch.float64)
    c = ctx.size(0)
    cache = [None] * dec.layers
    if c > 1:
        dec.forward(ctx[: c - 1], torch.arange(c - 1), cache)
    out = np.full(MAX_GEN, PAD, dtype=np.int32)
    x = ctx[c - 1]
    t = c - 1
    while True:
        h = dec.forward(x[None], torch.tensor([t]), cache)
        logp = F.log_softmax(dec.logits(h[0]), -1)
        token = int(logp.argmax())
        if margins is not None:
            top2 = torch.topk(logp, 2).values
            margins.append(float(top2[0] - top2[1]))
        out[t] = token
        done = token == EOS
        if t % CHECK_EVERY == 0 and t > c + CHECK_WINDOW:
            done |= compression_ratio(out[t - CHECK_WINDOW: t]) > CHECK_RATIO
        if done or t == limit:
            break
        x = dec.embed(token)
        t += 1
    return [int(v) for v in out[c - 1: t + 1] if v not in (PAD, BOS, EOS)]


@torch.inference_mode()
def beam_reference(dec: Fp64Decoder, ctx: torch.Tensor, beams: int, length_norm: bool = False,
                   limit: int = MAX_GEN - 4, margins: list | None = None, gaps: list | None = None) -> list[int]:
    """Beam search of one context [C, D] in the reference's order of computation (src/omniasr_trt/llm.py:205-254).

    ``beams`` hypotheses, each with its own K/V cache; at the first step only hypothesis 0 is live (the others
    score -1e6).  Every step a hypothesis offers score + log p for every token (``length_norm``: (score * c +
    log p) / (c + 1) with c its count of tokens other than PAD / EOS, used once hypothesis 0's count is above 0),
    a finished one only EOS at its frozen score; the best ``beams`` offers survive (sorted, ties to the lower
    flat index) and take their parents' caches, histories, scores and states.  The repetition stop ends the
    hypotheses whose last 100 tokens compress more than 4x at the checked positions.  The text is hypothesis 0's.
    Pinned by: one beam is ``greedy_reference``; with as many beams as tokens and a stop after two tokens, the
    result is the best of all two-token sequences by brute force (tests/test_oracle.py).

    ``margins``: if a list, receives per step the smallest gap between consecutive offers among the best
    ``beams`` + 1 finite ones (relative to their size): where it is tiny, another rounding of the same arithmetic
    can choose other survivors or order them differently.  ``gaps``: the same smallest gaps, absolute (in score
    units), for arithmetic whose error does not shrink with the scores' size (bf16 activations).
    """
    ctx = ctx.detach().to("cpu", torch.float64)
    c, n = ctx.size(0), beams
    caches = [[None] * dec.layers for _ in range(n)]
    if c > 1:
        dec.forward(ctx[: c - 1], torch.arange(c - 1), caches[0])
        for b in range(1, n):
            caches[b] = [(k.clone(), v.clone()) for k, v in caches[0]]
    out = np.full((n, MAX_GEN), PAD, dtype=np.int64)
    scores = np.full(n, -1e6)
    scores[0] = 0.0
    ended = np.zeros(n, dtype=bool)
    xs = [ctx[c - 1]] * n
    t = c - 1
    while True:
        logp = np.stack([F.log_softmax(dec.logits(dec.forward(xs[b][None], torch.tensor([t]), caches[b])[0]), -1)
                         .numpy() for b in range(n)])  # [n, V]
        count = ((out[:, :t] != PAD) & (out[:, :t] != EOS)).sum(1)[:, None]
        if length_norm and count[0, 0] > 0:
            cand = (scores[:, None] * count + logp) / (count + 1)
        else:
            cand = scores[:, None] + logp
        cand[ended] = -np.inf
        cand[ended, EOS] = scores[ended]
        flat = cand.reshape(-1)
        order = np.argsort(-flat, kind="stable")  # best first, ties to the lower flat index
        pick = order[:n]
        top = flat[pick]
        if margins is not None or gaps is not None:
            best = flat[order[: n + 1]]
            best = best[np.isfinite(best)]
            diffs = np.abs(np.diff(best))
            if margins is not None:
                rel = diffs / np.maximum(np.abs(best[1:]), 1.0)
                margins.append(float(rel.min()) if rel.size else math.inf)
            if gaps is not None:
                gaps.append(float(diffs.min()) if diffs.size else math.inf)
        parent, token = pick // cand.shape[1], pick % cand.shape[1]
        out, ended, scores = out[parent].copy(), ended[parent].copy(), scores[parent].copy()
        caches = [[(k.clone(), v.clone()) for k, v in caches[p]] for p in parent]
        scores = np.where(ended, scores, top)
        out[:, t] = token
        out[ended, t] = EOS
        ended = out[:, t] == EOS
        if t % CHECK_EVERY == 0 and t > c + CHECK_WINDOW:
            ended |= np.array([compression_ratio(row) > CHECK_RATIO for row in out[:, t - CHECK_WINDOW: t]])
        if ended.all() or t == limit:
            break
        xs = [dec.embed(int(out[b, t])) for b in range(n)]
        t += 1
    return [int(v) for v in out[0, c - 1: t + 1] if v not in (PAD, BOS, EOS)]

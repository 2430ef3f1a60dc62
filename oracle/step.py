"""A whole drafted decoder step in numpy (test infrastructure; see oracle/__init__.py).

``SpecDecoder.step`` (src/omniasr_trt/spec.py:82-108) restated over the oracle's kernels: proposal and step
assembly, embedding gather, per layer RMSNorm -> qkv GEMM -> RoPE + append -> causal multi-query attention -> output
projection -> RMSNorm -> gate|inner GEMM -> SiLU -> FFN output, final RMSNorm, LM head, log-softmax argmax and the
acceptance.  Everything in float32 (numpy has no bf16 GEMM).  ``bench.py`` times it on the host cores as the CPU
baseline of the verified-tokens/s metric.  Pinned by tests/test_oracle_step.py: on a small fp32 model, drafted
decoding with perfect, noisy and no drafts gives the fp64 reference-order loop's tokens, and every step's verify
logits agree with an fp64 forward over the same token sequence to fp32 precision.
"""

from __future__ import annotations

import numpy as np

from . import verify as ov

F32 = np.float32


def _rms(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    ms = np.mean(np.square(x, dtype=F32), axis=-1, keepdims=True, dtype=F32)
    return (x * (1.0 / np.sqrt(ms + F32(eps))).astype(F32) * w).astype(F32)


def _silu(x: np.ndarray) -> np.ndarray:
    return (x / (1.0 + np.exp(-x))).astype(F32)


class NumpySpecDecoder:
    """The drafted step over numpy copies of a decoder's weights, KV cache and per-slot state."""

    def __init__(self, weights: dict, num_layers: int, heads: int, eps: float, rope: np.ndarray, k_cache: np.ndarray,
                 v_cache: np.ndarray, state: dict, draft_tokens: int, ngram: int, behind: int, ahead: int, reach,
                 self_window: int, self_min: int, limit: int, eos: int):
        self.w = weights
        self.layers = num_layers
        self.heads = heads
        self.eps = eps
        self.rope = rope
        self.k, self.v = k_cache, v_cache  # [layers, B, H, S, D] float32
        self.s = state  # tok, last, done, out, draft, draft_len, next, first, start
        self.k_drafts = draft_tokens
        self.search = (ngram, behind, ahead, reach, 1 << (behind + ahead).bit_length(),
                       1 << (self_window - 1).bit_length(), self_min)
        self.limit, self.eos = limit, eos
        self.capacity = k_cache.shape[3]

    def step(self, keys: int) -> int:
        """One drafted step on every slot; returns the tokens accepted (sum over running rows of n + 1)."""
        s, w = self.s, self.w
        ngram, behind, ahead, reach, width, self_width, self_min = self.search
        t = self.k_drafts + 1
        tokens, pos, slots, lengths, use, start = ov.spec_prepare(
            s["out"], s["draft"], s["draft_len"], s["last"], s["first"], s["next"], s["tok"], s["done"],
            self.capacity, self.k_drafts, ngram, behind, ahead, reach, width, self_width, self_min)
        s["start"][:] = start
        h = w["text_frontend.weight"][tokens.reshape(-1)].astype(F32)
        scale = None
        for i in range(self.layers):
            p = f"llama_decoder.layers.{i}."
            qkv = _rms(h, w[p + "self_attn_layer_norm.weight"], self.eps) @ w[p + "qkv"].T
            q = ov.rope_kv(qkv, self.rope, pos, self.k[i], self.v[i], self.heads, slots, None, "f32")
            d = q.shape[-1]
            scale = d ** -0.5
            o = ov.verify_attention(q, self.k[i, :, :, :keys], self.v[i, :, :, :keys], lengths, t, scale)
            h = (h + o.astype(F32).reshape(h.shape[0], -1) @ w[p + "self_attn.output_proj.weight"].T).astype(F32)
            gi = _rms(h, w[p + "ffn_layer_norm.weight"], self.eps) @ w[p + "gi"].T
            gate, inner = np.split(gi, 2, axis=-1)
            h = (h + (inner * _silu(gate)) @ w[p + "ffn.output_proj.weight"].T).astype(F32)
        logits = _rms(h, w["llama_decoder.layer_norm.weight"], self.eps) @ w["final_proj.weight"].T
        self.last_logits, self.last_tokens = logits, tokens  # the step's verify logits [B*T, V] and fed tokens [B, T]
        nxt = ov.log_softmax_argmax(logits, "f32").reshape(-1, t)
        before = s["last"].copy()
        ov.accept(tokens, nxt, s["out"], s["tok"], s["last"], s["done"], s["next"], s["start"], use, self.limit,
                  self.eos)
        return int((s["last"] - before).sum())


def weights_from_state_dict(state_dict: dict) -> dict:
    """float32 numpy weights, with q|k|v and gate|inner concatenated as the decoders' fused GEMM operands."""
    w = {k: v.detach().float().cpu().numpy() for k, v in state_dict.items()}
    i = 0
    while f"llama_decoder.layers.{i}.self_attn.q_proj.weight" in w:
        p = f"llama_decoder.layers.{i}."
        w[p + "qkv"] = np.concatenate([w[p + f"self_attn.{x}_proj.weight"] for x in ("q", "k", "v")])
        w[p + "gi"] = np.concatenate([w[p + "ffn.gate_proj.weight"], w[p + "ffn.inner_proj.weight"]])
        for x in ("q", "k", "v"):
            del w[p + f"self_attn.{x}_proj.weight"]
        del w[p + "ffn.gate_proj.weight"], w[p + "ffn.inner_proj.weight"]
        i += 1
    return w

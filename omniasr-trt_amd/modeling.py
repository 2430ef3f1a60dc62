"""The omniASR LLM decoder (LLaMA) whose step the kernels serve: configuration, RoPE table, modules.

Module and parameter names are fairseq2's (``text_frontend``, ``llama_decoder.layers.{i}.self_attn.q_proj``,
... -- src/omniasr_trt/modeling.py:293-406), so the decoder part of an official checkpoint loads into
:class:`DecoderModel` unchanged.  The wav2vec2 encoder and the CTC head are not part of the decode step
and are not here: the step's inputs are decoder embeddings (a context of audio frames and text).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor, nn

HOP = 320  # samples per encoder frame at 16 kHz (20 ms)


@dataclass(frozen=True)
class DecoderConfig:
    """omniASR-LLM-7B's decoder (src/omniasr_trt/modeling.py:30-41)."""

    model_dim: int = 4096
    num_layers: int = 12
    num_heads: int = 8
    ffn_dim: int = 2816
    vocab_size: int = 10288
    # three marker ids after the vocabulary (language id, final segment, other segment): extra embedding rows
    num_special: int = 3
    num_langs: int = 1694
    max_seq_len: int = 8192
    rope_theta: float = 10_000.0
    rms_eps: float = 1e-5

    @property
    def head_dim(self) -> int:
        return self.model_dim // self.num_heads


# The synthetic benchmark stack: LLaMA-7B-like attention and FFN widths on the 12-layer omniASR decoder.
BENCH_CONFIG = DecoderConfig(model_dim=4096, num_layers=12, num_heads=32, ffn_dim=11008, vocab_size=10288)


def rope_table(cfg: DecoderConfig, device=None) -> Tensor:
    """cos/sin of every position, ``[max_seq_len, head_dim / 2, 2]`` fp32: pair j of position p rotates by
    p * theta^(-2j / head_dim) (fairseq2's RotaryEncoder; src/omniasr_trt/modeling.py:293-298)."""
    head_dim = cfg.head_dim
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim))
    angles = torch.outer(torch.arange(cfg.max_seq_len, device=device, dtype=torch.float32), inv)
    return torch.stack([torch.cos(angles), torch.sin(angles)], -1)


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: Tensor) -> Tensor:
        return F.rms_norm(x, (x.size(-1),), self.weight, self.eps)


class DecoderAttention(nn.Module):
    def __init__(self, cfg: DecoderConfig):
        super().__init__()
        d = cfg.model_dim
        self.heads = cfg.num_heads
        self.q_proj = nn.Linear(d, d, bias=False)
        self.k_proj = nn.Linear(d, d, bias=False)
        self.v_proj = nn.Linear(d, d, bias=False)
        self.output_proj = nn.Linear(d, d, bias=False)


class GLUFFN(nn.Module):
    def __init__(self, cfg: DecoderConfig):
        super().__init__()
        self.gate_proj = nn.Linear(cfg.model_dim, cfg.ffn_dim, bias=False)
        self.inner_proj = nn.Linear(cfg.model_dim, cfg.ffn_dim, bias=False)
        self.output_proj = nn.Linear(cfg.ffn_dim, cfg.model_dim, bias=False)


class DecoderLayer(nn.Module):
    def __init__(self, cfg: DecoderConfig):
        super().__init__()
        self.self_attn_layer_norm = RMSNorm(cfg.model_dim, cfg.rms_eps)
        self.self_attn = DecoderAttention(cfg)
        self.ffn_layer_norm = RMSNorm(cfg.model_dim, cfg.rms_eps)
        self.ffn = GLUFFN(cfg)


class LlamaDecoder(nn.Module):
    def __init__(self, cfg: DecoderConfig):
        super().__init__()
        self.layers = nn.ModuleList(DecoderLayer(cfg) for _ in range(cfg.num_layers))
        self.layer_norm = RMSNorm(cfg.model_dim, cfg.rms_eps)


class DecoderModel(nn.Module):
    """Text embeddings, language embeddings, the LLaMA decoder and the LM head of omniASR-LLM."""

    def __init__(self, dcfg: DecoderConfig = DecoderConfig()):
        super().__init__()
        self.dec_cfg = dcfg
        self.text_frontend = nn.Embedding(dcfg.vocab_size + dcfg.num_special, dcfg.model_dim)
        self.llama_decoder = LlamaDecoder(dcfg)
        self.final_proj = nn.Linear(dcfg.model_dim, dcfg.vocab_size, bias=False)
        self.lang_embeddings = nn.Embedding(dcfg.num_langs, dcfg.model_dim)
        self.register_buffer("rope", rope_table(dcfg), persistent=False)

    def _apply(self, fn, recurse=True):
        # .to / .cuda / .float / .double: the rotation table is recomputed in fp32 on the new device
        # (a cast would round it to the weights' dtype).
        out = super()._apply(fn, recurse)
        out.rope = rope_table(out.dec_cfg, out.rope.device)
        return out


def random_decoder(cfg: DecoderConfig, *, std: float = 0.02, seed: int = 0, dtype=torch.bfloat16,
                   device="cuda") -> DecoderModel:
    """A decoder with every weight N(0, std) (RMSNorm gains 1), drawn on ``device`` from a seeded generator --
    the random-init stack of the synthetic benchmarks (no checkpoint needed)."""
    with torch.device("meta"):
        m = DecoderModel(cfg)
    m = m.to_empty(device=device).to(dtype)
    g = torch.Generator(device=device).manual_seed(seed)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if name.endswith("layer_norm.weight"):
                p.fill_(1.0)
            else:
                p.normal_(0.0, std, generator=g)
    m.requires_grad_(False)
    m.rope = rope_table(cfg, device)
    return m.eval()


__all__ = ["BENCH_CONFIG", "DecoderConfig", "DecoderModel", "HOP", "RMSNorm", "random_decoder", "rope_table"]

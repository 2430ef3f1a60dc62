"""Batched greedy decoding of the omniASR LLM decoder on MI355X: static KV cache, HIP-graph steps, continuous
batching.

Behaviour of the reference's ``GreedyDecoder`` (src/omniasr_trt/decode.py): every slot (row of the batch) decodes
its own context at its own position; contexts of different lengths are prefilled together; a step feeds each
running slot's newest token, appends its K/V at the slot's position and attends to that slot's keys only (a finished
slot reads none); the host looks every ``sync_every`` steps -- EOS, the position cap, the zlib repetition stop, and a
new context for each slot whose context ended.

Slot state on the device, as the reference keeps it: ``out[r, t]`` is the token predicted from input position t,
``last[r]`` the position of the newest token ``tok[r]`` (the next step feeds it at ``last + 1``), ``done[r]`` marks a
finished slot.

A step is the HIP kernels of ``kernels`` (RoPE + KV append, verify attention, argmax + acceptance) between the
decoder's GEMMs, one HIP graph per (slots, key bucket).  There is no PyTorch attention or update path in the step.
"""

from __future__ import annotations

import os
from contextlib import nullcontext

import numpy as np
import torch
import torch.nn.functional as F
from torch import Tensor, nn
from torch.nn.utils.rnn import pad_sequence

from . import kernels
from .batching import GraphCache, UnitScheduler, packed_weights
from .llm import BOS, EOS, MAX_GEN, PAD, early_stop_index
from .modeling import DecoderModel

KEY_BUCKET = 256
LIMIT = MAX_GEN - 4  # the last input position the reference generates from
# Initial cache length.  A streaming context after an input's first segment holds two segments of audio frames, the
# previous segment's text and a few markers; starting at this size keeps those contexts from growing the caches (and
# re-capturing the graphs) call after call.
CONTEXT_FLOOR = 2048


def bucketed(n: int, bucket: int = KEY_BUCKET) -> int:
    """``n`` rounded up to a multiple of ``bucket``."""
    return -(-int(n) // bucket) * bucket


def fuse_projections(model: DecoderModel):
    """Per layer the four GEMM operands (q|k|v, attention output, gate|inner, FFN output) -- see
    :func:`batching.packed_weights`.  (src/omniasr_trt/decode.py:34-54)"""
    return packed_weights(model)


def _norm(norm: nn.Module, h: Tensor) -> Tensor:
    """A decoder RMSNorm on the residual rows: one HIP launch for bf16 rows on the GPU (``kernels.rms_norm``; model
    widths up to 8192), the module (torch) otherwise."""
    if kernels.rms_norm_supported(h, norm.weight):
        return kernels.rms_norm(h, norm.weight, norm.eps)
    return norm(h)


def _gated(gate_inner: Tensor) -> Tensor:
    """``inner * silu(gate)`` of the fused gate|inner projection: one HIP launch for bf16 rows on the GPU
    (``kernels.silu_mul``, torch's rounding), torch's two kernels otherwise."""
    if kernels.layer_ops_supported(gate_inner):
        return kernels.silu_mul(gate_inner)
    gate, inner = gate_inner.chunk(2, -1)
    return inner * F.silu(gate)


def _regrown(old: Tensor | None, shape: tuple, dim: int, fill, dtype, device) -> Tensor:
    """A new tensor of ``shape`` filled with ``fill`` that starts with ``old``'s contents along ``dim``."""
    new = torch.full(shape, fill, dtype=dtype, device=device)
    if old is not None:
        new.narrow(dim, 0, old.size(dim)).copy_(old)
    return new


class GreedyDecoder:
    """Greedy search with up to ``max_batch`` contexts in flight (the reference's constructor arguments)."""

    def __init__(self, model: DecoderModel, *, max_batch: int = 16, sync_every: int = 16, graphs: bool = True,
                 reserve: int = 768, fused: bool = True):
        if not fused:
            raise ValueError("this build has one decode path, the HIP kernels (fused=False is not available)")
        self.m = model
        self.dtype = model.final_proj.weight.dtype
        self.device = model.final_proj.weight.device
        if not kernels.available(self.device):
            raise RuntimeError(f"the decoder runs on the MI355X kernels: {self.device} is not a GPU device")
        cfg = model.dec_cfg
        self.fused = True
        self.layers = fuse_projections(model)
        self.heads = cfg.num_heads
        self.head_dim = cfg.model_dim // cfg.num_heads
        self.max_batch = max_batch
        self.sync_every = sync_every
        self.step_tokens = 1  # positions a slot can advance by in one step
        self.reserve = reserve  # positions beyond the longest context allocated up front
        self.context_floor = CONTEXT_FLOOR
        self.use_graphs = graphs
        self.graphs = GraphCache(self.device, graphs)
        # OMNIASR_TRT_DEBUG_SYNC=1: wait for the device after every stage, so an error names the stage that raised it
        self.debug_sync = os.environ.get("OMNIASR_TRT_DEBUG_SYNC") == "1"
        self.phase = lambda name: nullcontext()  # context manager per named stage; a profiling caller replaces it
        self.stats = {"steps": 0, "rows_steps": 0, "tokens": 0, "prefill_tokens": 0, "captures": 0, "grows": 0}
        self.capacity = 0
        self.k = self.v = self.out = None
        self._normal_capacity: int | None = None
        self._host: tuple | None = None  # (out, last) read back at the current look
        rows, dev = max_batch, self.device
        self.tok = torch.zeros(rows, dtype=torch.long, device=dev)
        self.last = torch.zeros(rows, dtype=torch.long, device=dev)
        self.done = torch.ones(rows, dtype=torch.bool, device=dev)
        # This decoder's own merge tickets of the attention (one per (row, head), zero between launches), so that
        # two decoders on different streams of one GPU never share them.
        self.attn_tickets = torch.zeros(rows * self.heads, dtype=torch.int32, device=dev)

    # ------------------------------------------------------------------ slot state kept across steps and graphs

    def ensure_capacity(self, length: int) -> None:
        """Make the KV cache and the token buffer hold ``length`` positions (rounded up to the key bucket, at most the
        position cap).  Growing keeps the contents and drops the graphs, which hold the old addresses."""
        target = min(bucketed(length), bucketed(MAX_GEN))
        if target <= self.capacity:
            return
        torch.cuda.synchronize(self.device)  # nothing in flight on the buffers being replaced
        kv_shape = (len(self.layers), self.max_batch, self.heads, target, self.head_dim)
        self.k = _regrown(self.k, kv_shape, 3, 0, self.dtype, self.device)
        self.v = _regrown(self.v, kv_shape, 3, 0, self.dtype, self.device)
        self.out = _regrown(self.out, (self.max_batch, target), 1, PAD, torch.int32, self.device)
        if self.capacity:
            self.stats["grows"] += 1
        self.capacity = target
        self.reset_graphs()

    def reset_graphs(self) -> None:
        self.graphs.clear()

    def release(self) -> None:
        """Free the KV cache and the graphs captured on it; the next call allocates its normal size again."""
        torch.cuda.synchronize(self.device)
        self.k = self.v = self.out = None
        self.capacity = 0
        self.reset_graphs()

    def check(self, where: str) -> None:
        if not self.debug_sync:
            return
        try:
            torch.cuda.synchronize(self.device)
        except Exception as e:
            raise RuntimeError(f"GPU error after {where} (capacity {self.capacity})") from e

    # ------------------------------------------------------------------ the decoder layers

    def _layer(self, i: int, h: Tensor, attend) -> None:
        """Decoder layer ``i`` on the residual stream ``h`` [N, D] in place; ``attend(qkv)`` returns the attention
        output [N, H*Dh] for the layer's q|k|v [N, 3*H*Dh] (it also writes the K/V cache)."""
        w = self.layers[i]
        layer = self.m.llama_decoder.layers[i]
        o = attend(_norm(layer.self_attn_layer_norm, h) @ w.qkv.t())
        h.addmm_(o, w.attn_out.t())  # the GEMM adds into the residual in place
        h.addmm_(_gated(_norm(layer.ffn_layer_norm, h) @ w.gate_inner.t()), w.ffn_out.t())

    def _head(self, h: Tensor) -> Tensor:
        return self.m.final_proj(_norm(self.m.llama_decoder.layer_norm, h))

    # ------------------------------------------------------------------ filling slots from their contexts

    def prefill(self, ctx: list[Tensor], slots: list[int] | None = None) -> Tensor:
        """Fill cache rows ``slots`` (default 0..B-1) with the contexts; returns each one's first token [B]."""
        return self.prefill_into(ctx, slots, self.k, self.v).argmax(-1)

    def prefill_into(self, ctx: list[Tensor], slots, k_cache: Tensor, v_cache: Tensor) -> Tensor:
        """The contexts (right-padded to the longest) through the decoder into rows ``slots`` of ``k_cache`` /
        ``v_cache`` ([layers, rows, H, S, Dh]); returns the log-softmax after each context's last token [B, V] in the
        model's dtype.  RoPE and the cache writes are ``kernels.rope_kv``; causal attention over each context is
        ``kernels.prefill_attention`` (bf16, head dim 128 / 256 / 512) or fp32 torch attention otherwise.  Padding
        comes after each context's tokens, and attention is causal, so no context position sees a pad.
        (src/omniasr_trt/decode.py:137-179)"""
        b = len(ctx)
        lens = torch.tensor([c.size(0) for c in ctx], device=self.device)
        width = int(lens.max())
        rows = torch.arange(b, device=self.device) if slots is None else torch.as_tensor(list(slots),
                                                                                           device=self.device)
        h = pad_sequence([c.to(self.dtype) for c in ctx], batch_first=True).reshape(b * width, -1).contiguous()
        pos = torch.arange(width, device=self.device).repeat(b)
        row_of = rows.repeat_interleave(width)
        scale = self.head_dim ** -0.5
        on_kernel = kernels.prefill_supported(self.dtype, self.head_dim)
        for i in range(len(self.layers)):
            kc, vc = k_cache[i], v_cache[i]

            def attend(qkv, kc=kc, vc=vc):
                q = kernels.rope_kv(qkv, self.m.rope, pos, kc, vc, self.heads, row_of)
                if on_kernel:
                    return kernels.prefill_attention(q, kc, vc, rows, width, scale).view(b * width, -1)
                # fp32 models and other head dims: torch attention in fp32 over the rows just written (fp32 keeps
                # bf16 batched products, and their transposed operands, out of this path)
                qf = q.view(b, width, self.heads, -1).transpose(1, 2).float()
                kf = kc[rows, :, :width].float()
                vf = vc[rows, :, :width].float()
                o = F.scaled_dot_product_attention(qf, kf, vf, is_causal=True).to(self.dtype)
                return o.transpose(1, 2).reshape(b * width, -1)

            self._layer(i, h, attend)
        final = h.view(b, width, -1)[torch.arange(b, device=self.device), lens - 1]
        self.stats["prefill_tokens"] += int(lens.sum())
        return F.log_softmax(self._head(final), dim=-1)

    # ------------------------------------------------------------------ the step over every slot

    def layer_stack(self, h: Tensor, pos: Tensor, slots: Tensor | None, lengths: Tensor, tokens: int,
                    keys: int) -> Tensor:
        """The decoder layers over the fed tokens ``h`` [B*T, D] (T = ``tokens`` per slot, at ``pos``, written to
        cache rows ``slots``, each slot's queries over its ``lengths`` keys plus the causal new ones); returns the
        LM-head logits [B*T, V]."""
        scale = self.head_dim ** -0.5
        n = h.size(0)
        for i in range(len(self.layers)):
            kc, vc = self.k[i], self.v[i]

            def attend(qkv, kc=kc, vc=vc):
                q = kernels.rope_kv(qkv, self.m.rope, pos, kc, vc, self.heads, slots)
                return kernels.draft_attention(q, kc, vc, lengths, tokens, keys, scale,
                                               tickets=self.attn_tickets).reshape(n, -1)

            self._layer(i, h, attend)
        return self._head(h)

    def step(self, b: int, keys: int) -> None:
        """One token for every running slot 0..b-1, in place; finished slots keep their state (they are fed again at
        their last position, read no keys, and nothing they produce is kept).  (src/omniasr_trt/decode.py:183-224)"""
        tok, last, done, out = self.tok[:b], self.last[:b], self.done[:b], self.out[:b]
        running = ~done
        p = last + running.long()
        lengths = torch.where(running, p + 1, 0)
        logits = self.layer_stack(self.m.text_frontend.weight[tok], p, None, lengths, 1, keys)
        kernels.greedy_accept(logits, tok[:, None], out, tok, last, done, None, None, None, LIMIT, EOS)

    def state(self) -> list[Tensor]:
        """The per-slot buffers a step changes besides the caches."""
        return [self.tok, self.last, self.done, self.out]

    def filled(self, slots: list[int], streams: list[int]) -> None:
        """Hook called after ``slots`` were given a context of ``streams`` (the drafted decoder loads drafts)."""

    def runner(self, b: int, keys: int):
        """The step of slots 0..b-1 with ``keys`` positions in reach, as a callable: a graph replay per (b, keys)."""
        before = self.graphs.captures
        run = self.graphs.runner((b, keys), lambda: self.step(b, keys), lambda: [t[:b] for t in self.state()])
        self.stats["captures"] += self.graphs.captures - before
        return run

    # ------------------------------------------------------------------ scheduling inputs onto slots

    @torch.inference_mode()
    def generate(self, contexts: list[Tensor]) -> list[list[int]]:
        """Greedy text tokens of each context (``[C, D]`` embeddings ending with <bos>)."""
        texts: list = [None] * len(contexts)

        def keep(j, tokens):
            texts[j] = tokens
            return None

        self.decode_streams(len(contexts), contexts.__getitem__, keep)
        return texts

    @torch.inference_mode()
    def decode_streams(self, n: int, start, advance) -> None:
        """Decode ``n`` independent streams of contexts, up to ``max_batch`` at once.  ``start(j)`` gives stream j's
        first context; ``advance(j, tokens)`` gets the greedy tokens of its current context and returns the next
        context, or None when the stream is over.  (src/omniasr_trt/decode.py:274-373)"""
        b = min(self.max_batch, n)
        # Idle slots run in the step graph too (reading no keys, writing at ``last``): park them at position 0, as a
        # previous call may have left positions past a cache released since.
        self.done[:b] = True
        self.last[:b] = 0
        self.tok[:b] = 0
        self._normal_capacity = None
        UnitScheduler(b, n, start, advance, admit=self._admit, finished=lambda: self._finished(b),
                      harvest=self._harvest, run_block=self._run_block, retire=self._retire).run()

    def _host_state(self, b: int) -> tuple[np.ndarray, np.ndarray]:
        """``out`` and ``last`` of slots 0..b-1 on the host, read once per look."""
        if self._host is None:
            self._host = (self.out[:b].cpu().numpy(), self.last[:b].cpu().numpy())
        return self._host

    def _finished(self, b: int) -> list[int]:
        self._host = None  # a new look
        return np.flatnonzero(self.done[:b].cpu().numpy()).tolist()

    def _admit(self, sched: UnitScheduler, pairs: list) -> None:
        """Prefill the contexts into their slots and start them: the prefill's argmax is the first token, predicted
        from the context's last position."""
        slots = [u for u, _, _ in pairs]
        ctxs = [c for _, _, c in pairs]
        others = [u for u in sched.active() if u not in set(slots)]
        want = max(max(c.size(0) for c in ctxs), self.context_floor) + self.reserve
        if others:  # slots still decoding must keep room for a whole block of steps
            lasts = self.last[torch.tensor(others, device=self.device)]
            want = max(want, int(lasts.max()) + self.sync_every * self.step_tokens + 2)
        self.ensure_capacity(want)
        if self._normal_capacity is None:
            self._normal_capacity = self.capacity
        with self.phase("prefill"):
            first = self.prefill(ctxs, slots)
        self.check("prefill")
        idx = torch.tensor(slots, device=self.device)
        pos = torch.tensor([c.size(0) - 1 for c in ctxs], device=self.device)
        self.out[idx] = PAD
        self.out[idx, pos] = first.to(torch.int32)
        self.tok[idx] = first
        self.last[idx] = pos
        self.done[idx] = (first == EOS) | (pos >= LIMIT)
        self.filled(slots, [j for _, j, _ in pairs])
        self._host = None

    def _harvest(self, sched: UnitScheduler, u: int) -> list[int]:
        """The tokens of slot u's finished context: predicted from its last context position up to its last
        position, or up to a repetition stop (that token kept); PAD / BOS / EOS dropped."""
        a = sched.assigned[u]
        out, last = self._host_state(sched.units)
        end = a.stop if a.stop >= 0 else int(last[u])
        self.stats["tokens"] += end - a.ctx_len + 2
        return [int(t) for t in out[u, a.ctx_len - 1: end + 1] if t not in (PAD, BOS, EOS)]

    def _run_block(self, sched: UnitScheduler) -> None:
        """``sync_every`` step replays on a key bucket that holds every active slot's keys after them, then the
        repetition check of each active slot up to its new position."""
        b = sched.units
        active = sched.active()
        _, last = self._host_state(b)
        need = int(max(last[u] for u in active)) + self.sync_every * self.step_tokens + 2
        if need > self.capacity:
            self.ensure_capacity(need + self.reserve)
            self.check("grow")
        run = self.runner(b, min(self.capacity, bucketed(need)))
        self.check("runner")
        for _ in range(self.sync_every):
            run()
            self.check("step")
        self.stats["steps"] += self.sync_every
        self.stats["rows_steps"] += self.sync_every * len(active)  # every active slot was running at the look
        self._host = None
        out, last = self._host_state(b)
        stopped = []
        for u in active:
            a = sched.assigned[u]
            if a.stop >= 0:
                continue
            hit = early_stop_index(out[u], a.checked + 1, int(last[u]), a.ctx_len)
            a.checked = int(last[u])
            if hit is not None:
                a.stop = hit
                stopped.append(u)
        if stopped:
            self.done[torch.tensor(stopped, device=self.device)] = True

    def _retire(self) -> None:
        # A long generation may have grown the cache (up to the position cap for every slot); a long-lived process
        # does not keep that: the next call starts from its normal size again.
        if self._normal_capacity is not None and self.capacity > self._normal_capacity:
            self.release()


__all__ = ["CONTEXT_FLOOR", "GreedyDecoder", "KEY_BUCKET", "LIMIT", "bucketed", "fuse_projections"]

"""Batched greedy decoding of the omniASR LLM decoder on MI355X: static KV cache, HIP graphs, host loop.

Behaviour of the reference's ``GreedyDecoder`` (src/omniasr_trt/decode.py): each slot (row) keeps its own
position; contexts of different lengths are prefilled together; a step writes each running row's K/V at its
own position and attends to its own keys only (finished rows read none); one step -- layers, LM head, argmax,
update -- is one HIP graph per (rows, key bucket), replayed ``sync_every`` times between two looks of the host
(EOS, the length cap, the zlib repetition stop, refilling finished slots with the next context).

State per slot: ``out[r, t]`` is the token predicted from input position t; ``last[r]`` is the position of the
newest token ``tok[r]``, which the next step feeds at ``last + 1``; ``done[r]`` marks a finished row.

The device work of a step is the HIP kernels of ``kernels`` (RoPE + KV append, verify attention, argmax +
acceptance) between the decoder's GEMMs; there is no PyTorch attention or update path.
"""

from __future__ import annotations

import os
from contextlib import nullcontext

import numpy as np
import torch
import torch.nn.functional as F
from torch import Tensor

from . import kernels
from .llm import BOS, EOS, MAX_GEN, PAD, early_stop_index
from .modeling import DecoderModel

KEY_BUCKET = 256
LIMIT = MAX_GEN - 4  # the reference stops after generating from this position
# The caches start this large so that contexts after a stream's first segment (two segments of audio, the
# previous text, markers) do not grow them -- and the graphs captured on them -- in every call.
CONTEXT_FLOOR = 2048


def fuse_projections(model: DecoderModel) -> list[tuple[Tensor, Tensor, Tensor, Tensor]]:
    """Per layer (qkv [3D, D], output [D, D], gate|inner [2F, D], ffn output [D, F]): q/k/v and gate/inner
    concatenated once into one GEMM operand each, the modules re-pointed at slices of them (no weight held
    twice)."""
    fused = []
    for layer in model.llama_decoder.layers:
        a, f = layer.self_attn, layer.ffn
        if not hasattr(layer, "_qkv"):
            with torch.no_grad():
                qkv = torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight])
                gi = torch.cat([f.gate_proj.weight, f.inner_proj.weight])
            d, n = a.q_proj.weight.size(0), f.gate_proj.weight.size(0)
            for j, p in enumerate((a.q_proj, a.k_proj, a.v_proj)):
                p.weight = torch.nn.Parameter(qkv[j * d: (j + 1) * d], requires_grad=False)
            f.gate_proj.weight = torch.nn.Parameter(gi[:n], requires_grad=False)
            f.inner_proj.weight = torch.nn.Parameter(gi[n:], requires_grad=False)
            layer._qkv, layer._gi = qkv, gi
        fused.append((layer._qkv, a.output_proj.weight, layer._gi, f.output_proj.weight))
    return fused


class GreedyDecoder:
    def __init__(self, model: DecoderModel, *, max_batch: int = 16, sync_every: int = 16, graphs: bool = True,
                 reserve: int = 768, fused: bool = True):
        self.m = model
        cfg = model.dec_cfg
        self.dtype = model.final_proj.weight.dtype
        self.device = model.final_proj.weight.device
        if not fused:
            raise ValueError("this build has one decode path, the HIP kernels (fused=False is not available)")
        if not kernels.available(self.device):
            raise RuntimeError(f"the decoder runs on the MI355X kernels: {self.device} is not a GPU device")
        self.fused = True
        self.layers = fuse_projections(model)
        self.heads = cfg.num_heads
        self.head_dim = cfg.model_dim // cfg.num_heads
        self.max_batch = max_batch
        self.sync_every = sync_every
        self.step_tokens = 1  # positions a row advances by at most in one step
        self.use_graphs = graphs
        self.debug_sync = os.environ.get("OMNIASR_TRT_DEBUG_SYNC") == "1"  # synchronise after each operation
        if self.use_graphs:
            self.pool = torch.cuda.graph_pool_handle()
            self.capture_stream = torch.cuda.Stream(self.device)
        self.reserve = reserve  # generated positions beyond the longest context before the cache grows
        self.context_floor = CONTEXT_FLOOR
        self.capacity = 0
        self.k = self.v = self.out = None
        self.graphs: dict = {}
        self.stats = {"steps": 0, "rows_steps": 0, "tokens": 0, "prefill_tokens": 0, "captures": 0, "grows": 0}
        b, dev = max_batch, self.device
        self.tok = torch.zeros(b, device=dev, dtype=torch.long)
        self.last = torch.zeros(b, device=dev, dtype=torch.long)
        self.done = torch.ones(b, device=dev, dtype=torch.bool)
        self.phase = lambda name: nullcontext()  # the transcriber's timer when profiling

    # ------------------------------------------------------------------ persistent buffers

    def ensure_capacity(self, length: int) -> None:
        """KV cache and token buffer for ``length`` positions (graphs hold their addresses, so they persist)."""
        length = min(-(-length // KEY_BUCKET) * KEY_BUCKET, -(-MAX_GEN // KEY_BUCKET) * KEY_BUCKET)
        if length <= self.capacity:
            return
        b, dev = self.max_batch, self.device
        torch.cuda.synchronize(dev)  # no step in flight while buffers and graphs are replaced
        shape = (len(self.layers), b, self.heads, length, self.head_dim)
        k = torch.zeros(shape, device=dev, dtype=self.dtype)
        v = torch.zeros(shape, device=dev, dtype=self.dtype)
        out = torch.full((b, length), PAD, device=dev, dtype=torch.int32)
        if self.capacity:
            k[..., : self.capacity, :] = self.k
            v[..., : self.capacity, :] = self.v
            out[:, : self.capacity] = self.out
            self.stats["grows"] += 1
        self.k, self.v, self.out, self.capacity = k, v, out, length
        self.reset_graphs()  # captured against the old buffers

    def check(self, where: str) -> None:
        if self.debug_sync:
            try:
                torch.cuda.synchronize(self.device)
            except Exception as e:
                raise RuntimeError(f"GPU error after {where} (capacity {self.capacity})") from e

    def reset_graphs(self) -> None:
        """Drop the captured graphs and start a new memory pool."""
        self.graphs.clear()
        if self.use_graphs:
            self.pool = torch.cuda.graph_pool_handle()

    def release(self) -> None:
        """Drop the KV cache and the graphs captured on it (the next call allocates its normal size again)."""
        torch.cuda.synchronize(self.device)
        self.k = self.v = self.out = None
        self.capacity = 0
        self.reset_graphs()

    # ------------------------------------------------------------------ prefill

    def prefill(self, ctx: list[Tensor], slots: list[int] | None = None) -> Tensor:
        """Fill cache rows ``slots`` (default 0..B-1) with the contexts; returns each one's first token [B]."""
        return self.prefill_into(ctx, slots, self.k, self.v).argmax(-1)

    def prefill_into(self, ctx: list[Tensor], slots, k_cache: Tensor, v_cache: Tensor) -> Tensor:
        """Contexts into rows ``slots`` of ``k_cache`` / ``v_cache`` ([layers, rows, H, S, Dh]) -- RoPE and the cache
        writes by ``kernels.rope_kv``, causal attention over each context by ``kernels.prefill_attention`` (bf16, head
        dim 128, 256 or 512; fp32 torch attention otherwise); returns the log-softmax after each context's last token [B, V]
        (model dtype).  (src/omniasr_trt/decode.py:137-179)"""
        m, b = self.m, len(ctx)
        lens = [c.size(0) for c in ctx]
        width = max(lens)
        rows = None if slots is None or list(slots) == list(range(b)) else torch.tensor(slots, device=self.device)
        x = torch.zeros(b, width, ctx[0].size(1), device=self.device, dtype=self.dtype)
        for j, c in enumerate(ctx):
            x[j, : lens[j]] = c
        h = x.view(b * width, -1)
        pos = torch.arange(width, device=self.device).repeat(b)
        ctx_rows = torch.arange(b, device=self.device) if rows is None else rows
        slot = ctx_rows.repeat_interleave(width)
        fused = kernels.prefill_supported(self.dtype, self.head_dim)
        for i, layer in enumerate(m.llama_decoder.layers):
            qkv_w, out_w, gi_w, ffo_w = self.layers[i]
            qkv = layer.self_attn_layer_norm(h) @ qkv_w.t()
            q = kernels.rope_kv(qkv, m.rope, pos, k_cache[i], v_cache[i], self.heads, slot)
            # Right padding and causal attention: no valid token sees a pad.
            if fused:  # bf16, head dim 128 / 256 / 512: the HIP causal attention over the cache rows just written
                o = kernels.prefill_attention(q, k_cache[i], v_cache[i], ctx_rows, width, self.head_dim ** -0.5)
                o = o.view(b * width, -1)
            else:  # fp32 math keeps bf16 batched products (and their transposed operands) out of this path
                q = q.view(b, width, self.heads, -1).transpose(1, 2)
                k = k_cache[i, :b, :, :width] if rows is None else k_cache[i, rows, :, :width]
                v = v_cache[i, :b, :, :width] if rows is None else v_cache[i, rows, :, :width]
                o = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=True).to(self.dtype)
                o = o.transpose(1, 2).reshape(b * width, -1)
            h.addmm_(o, out_w.t())  # in place: the GEMM adds into the residual, no copy of it
            gate, inner = (layer.ffn_layer_norm(h) @ gi_w.t()).chunk(2, -1)
            h.addmm_(inner * F.silu(gate), ffo_w.t())
        h = h.view(b, width, -1)
        last = h[torch.arange(b, device=self.device), torch.tensor(lens, device=self.device) - 1]
        logits = m.final_proj(m.llama_decoder.layer_norm(last))
        self.stats["prefill_tokens"] += sum(lens)
        return F.log_softmax(logits, dim=-1)

    # ------------------------------------------------------------------ one decode step

    def layer_stack(self, h: Tensor, pos: Tensor, slots: Tensor | None, lengths: Tensor, tokens: int,
                    keys: int) -> Tensor:
        """The decoder layers over the fed tokens ``h`` [B*T, D]; returns the LM-head logits [B*T, V]."""
        m = self.m
        scale = self.head_dim ** -0.5
        rows = h.size(0)
        for i, layer in enumerate(m.llama_decoder.layers):
            qkv_w, out_w, gi_w, ffo_w = self.layers[i]
            qkv = layer.self_attn_layer_norm(h) @ qkv_w.t()
            q = kernels.rope_kv(qkv, m.rope, pos, self.k[i], self.v[i], self.heads, slots)
            o = kernels.draft_attention(q, self.k[i], self.v[i], lengths, tokens, keys, scale).reshape(rows, -1)
            h.addmm_(o, out_w.t())  # in place: the GEMM adds into the residual, no copy of it
            gate, inner = (layer.ffn_layer_norm(h) @ gi_w.t()).chunk(2, -1)
            h.addmm_(inner * F.silu(gate), ffo_w.t())
        return m.final_proj(m.llama_decoder.layer_norm(h))

    def step(self, b: int, keys: int) -> None:
        """In place on rows 0..b-1 of the persistent buffers; finished rows are left as they are.
        (src/omniasr_trt/decode.py:183-224)"""
        tok, last, done, out = self.tok[:b], self.last[:b], self.done[:b], self.out[:b]
        running = ~done
        p = last + running.long()  # input position of ``tok``; finished rows recompute their last slot
        lengths = torch.where(running, p + 1, 0)  # finished rows read no keys (their outputs are not kept)
        h = self.m.text_frontend.weight[tok]  # [B, D]
        logits = self.layer_stack(h, p, None, lengths, 1, keys)
        kernels.greedy_accept(logits, tok[:, None], out, tok, last, done, None, None, None, LIMIT, EOS)

    def state(self) -> list[Tensor]:
        """The per-slot buffers a step changes (restored after the warm-up step of a capture)."""
        return [self.tok, self.last, self.done, self.out]

    def filled(self, slots: list[int], streams: list[int]) -> None:
        """Called after ``slots`` were prefilled with a context of ``streams`` (subclasses add their state)."""

    def runner(self, b: int, keys: int):
        """The step on rows 0..b-1 with ``keys`` cache positions in reach: a replayed HIP graph per (b, keys)."""
        if not self.use_graphs:
            return lambda: self.step(b, keys)
        key = (b, keys)
        if key not in self.graphs:
            # Captured by hand on a side stream into one shared pool; a warm-up step outside the capture first
            # (it also allocates what the kernels keep between calls), then the state it changed is restored
            # (the K/V it wrote are rewritten identically by the replay).
            torch.cuda.synchronize(self.device)
            saved = [t[:b].clone() for t in self.state()]
            stream = self.capture_stream
            stream.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(stream):
                self.step(b, keys)
                for t, v in zip(self.state(), saved, strict=True):
                    t[:b].copy_(v)
                graph = torch.cuda.CUDAGraph()
                graph.capture_begin(pool=self.pool)
                self.step(b, keys)
                graph.capture_end()
            torch.cuda.current_stream(self.device).wait_stream(stream)
            torch.cuda.synchronize(self.device)
            self.graphs[key] = graph
            self.stats["captures"] += 1
        return self.graphs[key].replay

    # ------------------------------------------------------------------ generate

    @torch.inference_mode()
    def generate(self, contexts: list[Tensor]) -> list[list[int]]:
        """Greedy text tokens of each context (``[C, D]`` embeddings ending with <bos>)."""
        results: list = [None] * len(contexts)

        def finish(j, tokens):
            results[j] = tokens
            return None

        self.decode_streams(len(contexts), contexts.__getitem__, finish)
        return results

    @torch.inference_mode()
    def decode_streams(self, n: int, start, advance) -> None:
        """Decode ``n`` independent streams of contexts with up to ``max_batch`` of them in flight.

        ``start(j)`` gives stream j's first context; ``advance(j, tokens)`` receives the greedy tokens of its current
        context and returns its next one (None: the stream is finished).  A slot whose context is finished takes its
        stream's next context (or a new stream) at the next host look, so the batch stays full.
        (src/omniasr_trt/decode.py:274-373)"""
        slots = _Slots(self, min(self.max_batch, n), iter(range(n)), start, advance)
        slots.run()


class _Slots:
    """Host side of ``decode_streams``: which stream each slot decodes and what the host has checked of it."""

    def __init__(self, dec: GreedyDecoder, b: int, upcoming, start, advance):
        self.dec, self.b = dec, b
        self.upcoming, self.start, self.advance = upcoming, start, advance
        self.stream = np.full(b, -1)  # stream decoded in each slot (-1: idle)
        self.ctx_len = np.zeros(b, dtype=np.int64)
        self.checked = np.zeros(b, dtype=np.int64)  # positions up to which the repetition check has run
        self.stopped = np.full(b, -1)  # position of a repetition stop
        self.normal: int | None = None

    def fill(self, pairs: list) -> None:
        """Prefill ``pairs`` [(slot, stream, context)] and reset those slots."""
        dec, b = self.dec, self.b
        refilled = {s for s, _, _ in pairs}
        in_flight = [int(dec.last[s]) for s in range(b) if self.stream[s] >= 0 and s not in refilled]
        longest = max(c.size(0) for _, _, c in pairs)
        dec.ensure_capacity(max([max(longest, dec.context_floor) + dec.reserve] +
                                [p + dec.sync_every * dec.step_tokens + 2 for p in in_flight]))
        self.normal = self.normal or dec.capacity
        slots = [s for s, _, _ in pairs]
        with dec.phase("prefill"):
            first = dec.prefill([c for _, _, c in pairs], slots)
        dec.check("prefill")
        idx = torch.tensor(slots, device=dec.device)
        pos = torch.tensor([c.size(0) - 1 for _, _, c in pairs], device=dec.device)
        dec.out[idx] = PAD
        dec.out[idx, pos] = first.to(torch.int32)
        dec.tok[idx] = first
        dec.last[idx] = pos
        dec.done[idx] = (first == EOS) | (pos >= LIMIT)
        for s, j, c in pairs:
            self.stream[s], self.ctx_len[s], self.checked[s], self.stopped[s] = j, c.size(0), c.size(0) - 1, -1
        dec.filled(slots, [j for _, j, _ in pairs])

    def finish(self, finished: list[int]) -> None:
        """Hand the tokens of finished slots to their streams and refill the slots."""
        dec = self.dec
        out = dec.out[: self.b].cpu().numpy()
        last = dec.last[: self.b].cpu().numpy()
        refill = []
        for s in finished:
            end = int(self.stopped[s]) if self.stopped[s] >= 0 else int(last[s])
            tokens = [int(t) for t in out[s, self.ctx_len[s] - 1: end + 1] if t not in (PAD, BOS, EOS)]
            dec.stats["tokens"] += end - int(self.ctx_len[s]) + 2
            j = int(self.stream[s])
            ctx = self.advance(j, tokens)
            if ctx is None:
                j = next(self.upcoming, None)
                ctx = None if j is None else self.start(j)
            self.stream[s] = -1
            if ctx is not None:
                refill.append((s, j, ctx))
        if refill:
            self.fill(refill)

    def run(self) -> None:
        dec, b = self.dec, self.b
        # Idle slots still run in the step graph (reading no keys) and write at their ``last`` position: reset it, as
        # a previous call may have left positions beyond a cache released since.
        dec.done[:b] = True
        dec.last[:b] = 0
        dec.tok[:b] = 0
        self.fill([(s, j, self.start(j)) for s, j in zip(range(b), self.upcoming)])
        while True:
            done = dec.done[:b].cpu().numpy()
            finished = [s for s in range(b) if self.stream[s] >= 0 and done[s]]
            if finished:
                self.finish(finished)
                continue  # a refilled slot may be finished at once (first token EOS)
            active = self.stream >= 0
            if not active.any():
                break
            last = dec.last[:b].cpu().numpy()
            need = int(last[active].max()) + dec.sync_every * dec.step_tokens + 2
            if need > dec.capacity:
                dec.ensure_capacity(need + dec.reserve)
                dec.check("grow")
            keys = min(dec.capacity, -(-need // KEY_BUCKET) * KEY_BUCKET)
            run = dec.runner(b, keys)
            dec.check("runner")
            for _ in range(dec.sync_every):
                run()
                dec.check("step")
            dec.stats["steps"] += dec.sync_every
            dec.stats["rows_steps"] += dec.sync_every * int((active & ~done).sum())
            self.repetition_check()
        if self.normal is not None and dec.capacity > self.normal:
            # A long generation grew the cache; a long-lived process must not keep that, so the next call starts
            # from its normal size again.
            dec.release()

    def repetition_check(self) -> None:
        dec, b = self.dec, self.b
        out = dec.out[:b].cpu().numpy()
        last = dec.last[:b].cpu().numpy()
        stop_now = []
        for s in range(b):
            if self.stream[s] < 0 or self.stopped[s] >= 0:
                continue
            hit = early_stop_index(out[s], int(self.checked[s]) + 1, int(last[s]), int(self.ctx_len[s]))
            self.checked[s] = last[s]
            if hit is not None:
                self.stopped[s] = hit
                stop_now.append(s)
        if stop_now:
            dec.done[torch.tensor(stop_now, device=dec.device)] = True


__all__ = ["CONTEXT_FLOOR", "GreedyDecoder", "KEY_BUCKET", "LIMIT", "fuse_projections"]

"""Host-side machinery shared by the decoders: packed projection weights, the cache of captured step graphs, and the
continuous-batching scheduler that keeps every decoding unit (a greedy slot, or a beam group) busy.

The scheduler owns only the control flow; what a unit is and how it runs belongs to the decoder, through four hooks
(see :class:`UnitScheduler`).  The flow is the one the reference's ``decode_streams`` loops follow
(src/omniasr_trt/decode.py:274-373, src/omniasr_trt/beam.py:216-315): admit a context per unit, replay a block of
steps, look at the device flags, hand finished units' tokens to their stream and give the unit the stream's next
context or a new stream, until no stream is left.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Iterator, NamedTuple

import torch
from torch import Tensor, nn


# ---------------------------------------------------------------------------------------------- packed GEMM operands

class LayerWeights(NamedTuple):
    """One decoder layer's GEMM operands ([out, in] each): q|k|v stacked, the attention output, gate|inner stacked,
    the FFN output."""

    qkv: Tensor
    attn_out: Tensor
    gate_inner: Tensor
    ffn_out: Tensor


def _stack_linears(module: nn.Module, names: tuple[str, ...]) -> Tensor:
    """The weights of ``module``'s Linear children ``names`` stacked along the output dimension into one tensor; the
    children are then given views into it, so the model keeps its fairseq2 parameter names and holds each weight
    once."""
    with torch.no_grad():
        stacked = torch.cat([getattr(module, name).weight for name in names], dim=0)
    offset = 0
    for name in names:
        linear = getattr(module, name)
        n = linear.weight.size(0)
        linear.weight = nn.Parameter(stacked.narrow(0, offset, n), requires_grad=False)
        offset += n
    return stacked


def packed_weights(model: nn.Module) -> list[LayerWeights]:
    """Per decoder layer, the operands of its four GEMMs (q|k|v and gate|inner each one GEMM), built once per model
    and cached on it.  (The reference's ``fuse_projections``, src/omniasr_trt/decode.py:34-54.)"""
    cached = model.__dict__.get("_omni_packed")
    if cached is None:
        cached = []
        for layer in model.llama_decoder.layers:
            attn, ffn = layer.self_attn, layer.ffn
            qkv = _stack_linears(attn, ("q_proj", "k_proj", "v_proj"))
            gate_inner = _stack_linears(ffn, ("gate_proj", "inner_proj"))
            cached.append(LayerWeights(qkv, attn.output_proj.weight, gate_inner, ffn.output_proj.weight))
        model.__dict__["_omni_packed"] = cached
    return cached


# ---------------------------------------------------------------------------------------------- step graphs

class GraphCache:
    """Captured HIP graphs of a decoder step, keyed by launch shape, all in one memory pool.

    A graph is captured by hand on a side stream (not ``torch.cuda.graph``, which empties the allocator's cache on
    every capture).  The step runs once outside the capture first -- it allocates what the kernels keep between
    calls, and a capture must not be the first call of the attention -- then the buffers that step changed are put
    back as they were, and the step is captured.  The warm-up's K/V writes are not undone: the replays write the
    same values to the same places.
    """

    def __init__(self, device: torch.device, enabled: bool):
        self.device = device
        self.enabled = enabled
        self.graphs: dict = {}
        self.captures = 0
        self.pool = torch.cuda.graph_pool_handle() if enabled else None
        self.stream = torch.cuda.Stream(device) if enabled else None

    def clear(self) -> None:
        """Forget every graph (the buffers they were captured on are being replaced) and start a new pool."""
        self.graphs.clear()
        if self.enabled:
            self.pool = torch.cuda.graph_pool_handle()

    def __len__(self) -> int:
        return len(self.graphs)

    def runner(self, key, step: Callable[[], None], mutated: Callable[[], list[Tensor]]) -> Callable[[], None]:
        """A callable running ``step`` once: the replay of its graph for ``key`` (captured on first use), or the
        eager step when graphs are off.  ``mutated()`` lists the tensors a step changes besides the caches."""
        if not self.enabled:
            return step
        graph = self.graphs.get(key)
        if graph is None:
            graph = self._capture(step, mutated)
            self.graphs[key] = graph
            self.captures += 1
        return graph.replay

    def _capture(self, step, mutated) -> torch.cuda.CUDAGraph:
        torch.cuda.synchronize(self.device)
        before = [t.clone() for t in mutated()]
        side, main = self.stream, torch.cuda.current_stream(self.device)
        side.wait_stream(main)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            step()
            for live, saved in zip(mutated(), before, strict=True):
                live.copy_(saved)
            graph.capture_begin(pool=self.pool)
            step()
            graph.capture_end()
        main.wait_stream(side)
        torch.cuda.synchronize(self.device)
        return graph


# ---------------------------------------------------------------------------------------------- scheduler

@dataclass
class Assignment:
    """What a unit decodes: ``stream``'s current context of ``ctx_len`` positions.  ``checked`` and ``stop`` are the
    greedy slots' repetition-check bookkeeping (last position checked, position of a repetition stop or -1)."""

    stream: int
    ctx_len: int
    checked: int = 0
    stop: int = -1


class UnitScheduler:
    """Runs ``n_streams`` streams of contexts over ``units`` decoding units.

    ``start(j)`` returns stream j's first context; ``advance(j, tokens)`` takes the tokens of its current context and
    returns its next context or None (the stream is over).  The decoder supplies:

    * ``admit(scheduler, pairs)`` -- prefill ``[(unit, stream, context)]`` and set those units decoding (their
      :class:`Assignment` is already in ``assigned``);
    * ``finished()`` -- units whose current decode has ended (reads the device flags);
    * ``harvest(scheduler, unit)`` -- the tokens of a finished unit's context;
    * ``run_block(scheduler)`` -- replay the next block of steps on every unit, with the host checks that follow it;
    * ``retire()`` -- called once when every stream is over.

    The hooks get the scheduler as an argument rather than holding it, so no reference cycle keeps a decoder (and
    the graphs it captured) alive after a call.

    A unit whose context ends hands its tokens on at the next look and takes the stream's next context (or the next
    stream), so the batch stays full instead of waiting for its slowest row.
    """

    def __init__(self, units: int, n_streams: int, start, advance, *, admit, finished, harvest, run_block,
                 retire=lambda: None):
        self.units = units
        self.pending: Iterator[int] = iter(range(n_streams))
        self.start, self.advance = start, advance
        self.assigned: list[Assignment | None] = [None] * units
        self._admit, self._finished, self._harvest = admit, finished, harvest
        self._run_block, self._retire = run_block, retire

    def active(self) -> list[int]:
        return [u for u, a in enumerate(self.assigned) if a is not None]

    def _next_stream(self) -> tuple[int, Tensor] | None:
        j = next(self.pending, None)
        return None if j is None else (j, self.start(j))

    def assign(self, pairs: list) -> None:
        """Record the units' new assignments and admit their contexts."""
        for unit, stream, ctx in pairs:
            n = ctx.size(0)
            self.assigned[unit] = Assignment(stream, n, checked=n - 1)
        self._admit(self, pairs)

    def run(self) -> None:
        first = []
        for unit in range(self.units):
            nxt = self._next_stream()
            if nxt is None:
                break
            first.append((unit, *nxt))
        if first:
            self.assign(first)
        while True:
            ended = [u for u in self._finished() if self.assigned[u] is not None]
            if ended:
                self._rotate(ended)
                continue  # a unit just admitted may have ended at once (first token EOS)
            if not self.active():
                break
            self._run_block(self)
        self._retire()

    def _rotate(self, ended: list[int]) -> None:
        """Hand the ended units' tokens on and give each the next context of its stream, or a new stream."""
        refill = []
        for unit in ended:
            a = self.assigned[unit]
            following = self.advance(a.stream, self._harvest(self, unit))
            self.assigned[unit] = None
            if following is not None:
                refill.append((unit, a.stream, following))
            else:
                nxt = self._next_stream()
                if nxt is not None:
                    refill.append((unit, *nxt))
        if refill:
            self.assign(refill)


__all__ = ["Assignment", "GraphCache", "LayerWeights", "UnitScheduler", "packed_weights"]

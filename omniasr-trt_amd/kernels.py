"""The decode-step kernels of the omniASR LLM decoder on MI355X (gfx950), behind omniasr-trt's API.

Same functions, arguments and results as ``omniasr_trt.kernels`` (src/omniasr_trt/kernels.py), so the
decoders above it are unchanged; each one calls a hand-written HIP kernel of ``libomniasr_mi355x.so``
through its C ABI (``include/omniasr_mi355x.h``) on torch's current stream:

* :func:`rope_kv` -- RoPE of q and k at each token's position, k and v written into the KV cache
  (``omni_rope_kv_append``);
* :func:`draft_attention` -- the verify attention of a drafted step: a row's T queries over its own
  keys, causal among the new ones, one read of the keys for all of them; :func:`decode_attention` is
  its one-query case (``omni_verify_attention``);
* :func:`propose` -- the draft proposal of every row (``omni_propose``);
* :func:`accept` -- greedy acceptance and rollback (``omni_accept``);
* :func:`beam_attention` -- beam search's shared-context plus generated-keys attention (``omni_beam_attention``);
  with a :class:`GenList` from :func:`beam_gen_list` (no counterpart in the reference) each generated key the beams
  of a group share is read once (``omni_beam_gen_list``, ``omni_beam_attention_listed``).

Beyond the reference's functions, for the fused step: :func:`spec_prepare` (proposal plus the step's
tokens / positions / cache rows / key counts in one launch) and :func:`greedy_accept` (the argmax of
the verify logits and the acceptance); for the prefill: :func:`prefill_attention` (causal attention of whole
contexts, the reference's ``F.scaled_dot_product_attention(is_causal=True)``).

Nothing here synchronises or allocates beyond the outputs and the attention workspace (from torch's
allocator, so from a graph's pool under capture), so every function can be captured in a HIP graph.  There is
no other code path: on a GPU without the library these functions raise.
"""

from __future__ import annotations

import ctypes

import torch
import torch.nn.functional as F

from . import _lib

# Launch settings of draft_attention / decode_attention.  ``split_k``: always plain split-K (otherwise the library
# runs the balanced halves kernel for head dim 128 when rows x heads cover the CUs, and for head dims 256 / 512 a
# split-K whose workgroup budget is dealt to the rows by length, merged in the kernel).  Plain split-K only: ``chunk``
# keys per split (0: the library's choice for the launch shape), ``separate``: merge the splits in a second launch
# (else the last split of each row and head merges them, reading the other splits' partials at the coherence point).
DRAFT_ATTN = {"chunk": 0, "separate": True, "split_k": False}
ATTN = {"chunk": 0, "separate": True, "split_k": False}

_counters: dict[int, torch.Tensor] = {}
_select_tickets: dict[int, torch.Tensor] = {}
# Ticket buffers replaced by larger ones: captured graphs may still hold their addresses, so they
# live as long as the process.
_retired: list[torch.Tensor] = []


def available(device: torch.device) -> bool:
    """True on a GPU device (the library is loaded; a missing library raises), False elsewhere."""
    device = torch.device(device)
    if device.type != "cuda":
        return False
    _lib.load()
    return True


def _dtype(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return _lib.BF16
    if t.dtype == torch.float32:
        return _lib.F32
    raise TypeError(f"the HIP kernels take bfloat16 or float32, not {t.dtype}")


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def _need(cond: bool, what: str) -> None:
    if not cond:
        raise ValueError(what)


def _index(t: torch.Tensor, name: str) -> None:
    _need(t.dtype == torch.long and t.is_contiguous() and t.is_cuda, f"{name}: contiguous int64 on the GPU")


def next_power_of_2(n: int) -> int:
    return 1 if n <= 1 else 1 << (int(n) - 1).bit_length()


def rope_kv(qkv: torch.Tensor, cs: torch.Tensor, pos: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
            heads: int, slots: torch.Tensor | None = None, cache_pos: torch.Tensor | None = None) -> torch.Tensor:
    """``qkv`` [N, 3*H*D] (q|k|v of N tokens), ``cs`` [P, D/2, 2] fp32, ``pos`` [N]; ``k_cache``/``v_cache``
    [rows, H, S, D] with unit stride in D.  Rotates at ``pos[n]`` and writes token n's k, v at cache row
    ``slots[n]`` (default n), position ``cache_pos[n]`` (default ``pos[n]``); returns the rotated q [N, H, D].
    (src/omniasr_trt/kernels.py:294-306)"""
    lib = _lib.load()
    n = qkv.size(0)
    dim = qkv.size(1) // (3 * heads)
    _need(qkv.dim() == 2 and qkv.stride(1) == 1, "qkv: [N, 3*H*D] with unit stride in the last dimension")
    _need(k_cache.dtype == qkv.dtype == v_cache.dtype, "qkv and the caches: one dtype")
    _need(k_cache.stride() == v_cache.stride() and k_cache.shape == v_cache.shape, "k_cache / v_cache: same layout")
    _need(k_cache.dim() == 4 and k_cache.stride(3) == 1 and k_cache.size(3) == dim, "caches: [rows, H, S, D]")
    _need(cs.dtype == torch.float32 and cs.is_contiguous() and cs.size(-2) * 2 == dim, "cs: [P, D/2, 2] fp32")
    _index(pos, "pos")
    for name, t in (("slots", slots), ("cache_pos", cache_pos)):
        if t is not None:
            _index(t, name)
    q = torch.empty(n, heads, dim, device=qkv.device, dtype=qkv.dtype)
    status = lib.omni_rope_kv_append(
        qkv.data_ptr(), qkv.stride(0), cs.data_ptr(), cs.size(0), pos.data_ptr(), _ptr(slots), _ptr(cache_pos),
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1),
        k_cache.stride(2), k_cache.size(0), k_cache.size(2), n, heads, dim, _dtype(qkv), _stream(qkv))
    _lib.check(status, "rope_kv")
    return q


def _tickets(store: dict, device: torch.device, n: int, what: str, least: int) -> torch.Tensor:
    """At least ``n`` int32 tickets on ``device`` from ``store``: zero, and left zero by every call."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    have = store.get(idx)
    if have is None or have.numel() < n:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"{what}: its tickets must be allocated before graph capture "
                               "(run the step once outside the capture)")
        size = max(n, least, 0 if have is None else 2 * have.numel())
        if have is not None:
            _retired.append(have)
        store[idx] = have = torch.zeros(size, device=device, dtype=torch.int32)
    return have


def _attn_counters(device: torch.device, n: int) -> torch.Tensor:
    """Per-(row, head) tickets of the split merge."""
    return _tickets(_counters, device, n, "verify attention", 1 << 16)


def _own_tickets(tickets: torch.Tensor | None, device: torch.device, n: int) -> torch.Tensor:
    """A caller's merge tickets (zero, at least ``n`` int32 on ``device``, left zero by every call), or the shared
    per-device ones.  Calls that share tickets must not overlap in time: a caller that runs on its own stream beside
    others (each decoder) passes its own."""
    if tickets is None:
        return _attn_counters(device, n)
    _need(tickets.dtype == torch.int32 and tickets.is_contiguous() and tickets.device == device
          and tickets.numel() >= n, f"tickets: at least {n} contiguous int32 on {device}")
    return tickets


def _verify(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, lengths: torch.Tensor, tokens: int,
            keys: int, scale: float, chunk: int, separate: bool, split_k: bool = False,
            tickets: torch.Tensor | None = None) -> torch.Tensor:
    lib = _lib.load()
    rows_total, heads, dim = q.shape
    _need(rows_total % tokens == 0, "q: [B*T, H, D]")
    groups = rows_total // tokens
    _need(q.is_contiguous(), "q: contiguous [B*T, H, D]")
    _need(k_cache.dtype == q.dtype == v_cache.dtype, "q and the caches: one dtype")
    _need(k_cache.stride() == v_cache.stride() and k_cache.shape == v_cache.shape, "k_cache / v_cache: same layout")
    _need(k_cache.dim() == 4 and k_cache.stride(3) == 1 and k_cache.size(3) == dim, "caches: [>=B, H, S, D]")
    _need(k_cache.size(0) >= groups and k_cache.size(1) == heads, "caches: at least B rows of H heads")
    _index(lengths, "lengths")
    _need(lengths.numel() >= groups, "lengths: [B]")
    chunk = int(chunk or 0)
    ws = lib.omni_verify_attention_workspace(groups, tokens, heads, dim, keys, chunk)
    workspace = torch.empty(max(ws, 256), device=q.device, dtype=torch.uint8)
    counters = _own_tickets(tickets, q.device, groups * heads)
    out = torch.empty_like(q)
    flags = (_lib.ATTN_SEPARATE_COMBINE if separate else 0) | (_lib.ATTN_SPLIT_K if split_k else 0)
    status = lib.omni_verify_attention(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1),
        k_cache.stride(2), k_cache.size(2), lengths.data_ptr(), groups, tokens, heads, dim, keys, chunk,
        float(scale), out.data_ptr(), workspace.data_ptr(), workspace.numel(), counters.data_ptr(), flags,
        _dtype(q), _stream(q))
    _lib.check(status, "verify attention")
    return out


_static_ready: set[int] = set()


def static_init(device: torch.device) -> None:
    """Set-up of :func:`verify_attention_static` on ``device`` (``omni_verify_attention_static_init``, once per
    device, outside graph capture): the library's static scratch gets its device address."""
    device = torch.device(device)
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx in _static_ready:
        return
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("verify_attention_static: call kernels.static_init(device) before graph capture")
    with torch.cuda.device(idx):
        _lib.check(_lib.load().omni_verify_attention_static_init(), "verify attention static scratch set-up")
    _static_ready.add(idx)


def verify_attention_static(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, lengths: torch.Tensor,
                            tokens: int, keys: int, scale: float, out: torch.Tensor, chunk: int = 0,
                            separate: bool = True, split_k: bool = False) -> torch.Tensor:
    """:func:`draft_attention` into the caller's ``out`` (same shape and dtype as ``q``) with nothing allocated: the
    library's per-GPU static scratch holds the split partials and tickets (``omni_verify_attention_static``).  Shapes
    whose workspace exceeds ``_lib.STATIC_WORKSPACE_BYTES`` (or with rows x heads > ``_lib.STATIC_MAX_UNITS``) raise.
    Calls that overlap in time on one GPU race: they share its scratch.  The scratch's address is looked up by the
    first call on each device (``omni_verify_attention_static_init``), which must not be under graph capture."""
    lib = _lib.load()
    static_init(q.device)
    rows_total, heads, dim = q.shape
    _need(rows_total % tokens == 0, "q: [B*T, H, D]")
    groups = rows_total // tokens
    _need(q.is_contiguous(), "q: contiguous [B*T, H, D]")
    _need(out.shape == q.shape and out.dtype == q.dtype and out.is_contiguous() and out.device == q.device,
          "out: contiguous, q's shape, dtype and device")
    _need(k_cache.dtype == q.dtype == v_cache.dtype, "q and the caches: one dtype")
    _need(k_cache.stride() == v_cache.stride() and k_cache.shape == v_cache.shape, "k_cache / v_cache: same layout")
    _need(k_cache.dim() == 4 and k_cache.stride(3) == 1 and k_cache.size(3) == dim, "caches: [>=B, H, S, D]")
    _need(k_cache.size(0) >= groups and k_cache.size(1) == heads, "caches: at least B rows of H heads")
    _index(lengths, "lengths")
    _need(lengths.numel() >= groups, "lengths: [B]")
    flags = (_lib.ATTN_SEPARATE_COMBINE if separate else 0) | (_lib.ATTN_SPLIT_K if split_k else 0)
    status = lib.omni_verify_attention_static(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1),
        k_cache.stride(2), k_cache.size(2), lengths.data_ptr(), groups, tokens, heads, dim, keys, int(chunk or 0),
        float(scale), out.data_ptr(), flags, _dtype(q), _stream(q))
    _lib.check(status, "verify attention (static scratch)")
    return out


def draft_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, lengths: torch.Tensor,
                    tokens: int, keys: int, scale: float, *, tickets: torch.Tensor | None = None,
                    **launch) -> torch.Tensor:
    """Draft verification: ``q`` [B*T, H, D], row b's T queries at rows b*T .. b*T+T-1; query i of row b attends to
    keys [0, lengths[b] + i) of cache row b (``k_cache``/``v_cache`` [>=B, H, S, D], all within the first ``keys``).
    One K/V read serves all T queries of a row.  Returns [B*T, H, D] in q's dtype.  ``launch``: overrides of
    ``DRAFT_ATTN`` (the reference's Triton settings -- block, warps, stages, programs -- have no meaning here and
    are ignored).  ``tickets``: the caller's own merge tickets (B*H int32, zero; see :func:`_own_tickets`).
    (src/omniasr_trt/kernels.py:338-358)"""
    cfg = {**DRAFT_ATTN, **{k: v for k, v in launch.items() if k in DRAFT_ATTN}}
    return _verify(q, k_cache, v_cache, lengths, tokens, keys, scale, cfg["chunk"], cfg["separate"], cfg["split_k"],
                   tickets)


def decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, lengths: torch.Tensor,
                     keys: int, scale: float, block: int | None = None, warps: int | None = None,
                     stages: int | None = None, programs: int | None = None, chunk: int | None = None, *,
                     tickets: torch.Tensor | None = None) -> torch.Tensor:
    """``q`` [B, H, D]; ``k_cache``/``v_cache`` [>=B, H, S, D]; row r attends to keys [0, lengths[r]) (all within the
    first ``keys``, which fixes the launch grid).  Returns [B, H, D] in q's dtype.  ``block`` / ``warps`` /
    ``stages`` / ``programs`` are the reference's Triton settings, accepted and ignored.
    (src/omniasr_trt/kernels.py:406-423)"""
    del block, warps, stages, programs
    return _verify(q, k_cache, v_cache, lengths, 1, keys, scale, ATTN["chunk"] if chunk is None else chunk,
                   ATTN["separate"], ATTN["split_k"], tickets)


class GenList:
    """Each group's generated keys listed once per distinct (row, position) -- ``offsets`` [S, N*G] uint32 (as
    int32), ``masks`` [S, N*G] uint16 (as int16), ``counts`` [S] int32 -- built by :func:`beam_gen_list` from one
    step's pointers and lengths for generated caches of one layout; :func:`beam_attention` reads it."""

    def __init__(self, groups: int, beams: int, gen_cap: int, device):
        self.stride = beams * gen_cap
        self.offsets = torch.empty(groups, self.stride, dtype=torch.int32, device=device)
        self.masks = torch.empty(groups, self.stride, dtype=torch.int16, device=device)
        self.counts = torch.zeros(groups, dtype=torch.int32, device=device)
        self.groups, self.beams, self.gen_cap = groups, beams, gen_cap
        self.layout = None  # (strides, rows) of the generated caches the offsets address


def beam_gen_list(lst: GenList, ptr: torch.Tensor, gen_len: torch.Tensor, kg: torch.Tensor, groups: int) -> GenList:
    """Fill ``lst`` for groups 0..groups-1 from ``ptr`` [>=S*N, >=G] int32 and ``gen_len`` [>=S*N] (as for
    :func:`beam_attention`), for generated caches laid out as ``kg`` [rows, H, G, D] (every layer's cache of one
    decoder shares the layout).  One launch; the beams of a group share most generated keys, and the attention then
    reads each of them once.  No counterpart in the reference."""
    lib = _lib.load()
    _need(0 < groups <= lst.groups and kg.size(2) == lst.gen_cap, "list: groups and generated capacity")
    _need(ptr.dtype == torch.int32 and ptr.dim() == 2 and ptr.stride(1) == 1 and ptr.size(1) >= kg.size(2),
          "ptr: [>=S*N, >=G] int32 with unit stride in positions")
    _index(gen_len, "gen_len")
    _need(ptr.size(0) >= groups * lst.beams and gen_len.numel() >= groups * lst.beams, "ptr / gen_len: S*N rows")
    status = lib.omni_beam_gen_list(groups, lst.beams, ptr.data_ptr(), ptr.stride(0), gen_len.data_ptr(), kg.size(2),
                                    kg.size(0), kg.stride(0), kg.stride(2), lst.offsets.data_ptr(),
                                    lst.masks.data_ptr(), lst.counts.data_ptr(), lst.stride, _stream(kg))
    _lib.check(status, "beam generated-key list")
    lst.layout = (kg.stride(), kg.size(0))
    return lst


def beam_attention(q: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, ctx_len: torch.Tensor, kg: torch.Tensor,
                   vg: torch.Tensor, ptr: torch.Tensor, gen_len: torch.Tensor, beams: int, ctx_keys: int,
                   scale: float, chunk: int = 0, gen_list: GenList | None = None,
                   tickets: torch.Tensor | None = None) -> torch.Tensor:
    """Beam rows ``q`` [S*N, H, D] (input g's beams are rows g*N .. g*N+N-1): attention over input g's context
    ``kc``/``vc`` [>=S, H, C, D] (first ``ctx_len[g]`` keys, all within ``ctx_keys``) and row r's generated keys
    ``kg``/``vg`` [>=S*N, H, G, D], position j read from row ``ptr[r, j]`` (first ``gen_len[r]``).  One pass over
    a group's context serves all of its beams.  Returns [S*N, H, D] in q's dtype.  ``gen_list``: the step's
    :func:`beam_gen_list` of the same pointers and lengths (optional; each shared generated key is then read once).
    ``tickets``: the caller's own merge tickets (S*H int32, zero; see :func:`_own_tickets`).
    (src/omniasr_trt/kernels.py:309-332)"""
    lib = _lib.load()
    rows, heads, dim = q.shape
    _need(beams >= 1 and rows % beams == 0, "q: [S*N, H, D]")
    groups = rows // beams
    _need(q.is_contiguous(), "q: contiguous [S*N, H, D]")
    for name, a, b in (("kc / vc", kc, vc), ("kg / vg", kg, vg)):
        _need(a.dtype == q.dtype == b.dtype, f"q and {name}: one dtype")
        _need(a.stride() == b.stride() and a.shape == b.shape, f"{name}: same layout")
        _need(a.dim() == 4 and a.stride(3) == 1 and a.size(3) == dim and a.size(1) == heads,
              f"{name}: [rows, H, positions, D] with unit stride in D")
    _need(kc.size(0) >= groups, "kc: at least S rows")
    _need(kg.size(0) >= rows, "kg: at least S*N rows")
    _need(ptr.dtype == torch.int32 and ptr.dim() == 2 and ptr.stride(1) == 1 and ptr.size(0) >= rows
          and ptr.size(1) >= kg.size(2), "ptr: [>=S*N, >=G] int32 with unit stride in positions")
    _index(ctx_len, "ctx_len")
    _index(gen_len, "gen_len")
    _need(ctx_len.numel() >= groups and gen_len.numel() >= rows, "ctx_len: [S], gen_len: [S*N]")
    ws = lib.omni_beam_attention_workspace(groups, beams, heads, dim, ctx_keys, int(chunk))
    workspace = torch.empty(max(ws, 256), device=q.device, dtype=torch.uint8)
    counters = _own_tickets(tickets, q.device, groups * heads)
    out = torch.empty_like(q)
    args = (q.data_ptr(), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2), kc.size(2),
            ctx_len.data_ptr(), kg.data_ptr(), vg.data_ptr(), kg.stride(0), kg.stride(1), kg.stride(2), kg.size(2),
            kg.size(0), ptr.data_ptr(), ptr.stride(0), gen_len.data_ptr())
    tail = (groups, beams, heads, dim, int(ctx_keys), int(chunk), float(scale), out.data_ptr(), workspace.data_ptr(),
            workspace.numel(), counters.data_ptr(), _dtype(q), _stream(q))
    if gen_list is None:
        status = lib.omni_beam_attention(*args, *tail)
    else:
        _need(gen_list.beams == beams and gen_list.groups >= groups and gen_list.layout == (kg.stride(), kg.size(0)),
              "gen_list: built by beam_gen_list for these beams and generated caches")
        status = lib.omni_beam_attention_listed(*args, gen_list.offsets.data_ptr(), gen_list.masks.data_ptr(),
                                                gen_list.counts.data_ptr(), gen_list.stride, *tail)
    _lib.check(status, "beam attention")
    return out


def prefill_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, slots: torch.Tensor,
                      width: int, scale: float) -> torch.Tensor:
    """Causal attention of whole contexts over their cache rows: ``q`` [B*width, H, D] bf16, D = 128, 256 or 512
    (context b's queries at rows b*width ..), ``k_cache``/``v_cache``
    [rows, H, S >= width, D] bf16 with unit stride in D, ``slots`` [B]
    the contexts' cache rows; query p of context b attends to keys [0, p] of row ``slots[b]``.  Returns
    [B*width, H, D] -- ``F.scaled_dot_product_attention(q, k, v, is_causal=True)`` of the prefill
    (src/omniasr_trt/decode.py:163-164), in the query layout of :func:`rope_kv`."""
    lib = _lib.load()
    rows, heads, dim = q.shape
    _need(width > 0 and rows % width == 0, "q: [B*width, H, D]")
    contexts = rows // width
    _need(q.is_contiguous(), "q: contiguous [B*width, H, D]")
    _need(k_cache.dtype == q.dtype == v_cache.dtype, "q and the caches: one dtype")
    _need(k_cache.stride() == v_cache.stride() and k_cache.shape == v_cache.shape, "k_cache / v_cache: same layout")
    _need(k_cache.dim() == 4 and k_cache.stride(3) == 1 and k_cache.size(3) == dim and k_cache.size(1) == heads,
          "caches: [rows, H, S, D] with unit stride in D")
    _need(k_cache.size(2) >= width, "caches: at least width positions")
    _index(slots, "slots")
    _need(slots.numel() >= contexts, "slots: [B]")
    out = torch.empty_like(q)
    status = lib.omni_prefill_attention(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1),
        k_cache.stride(2), k_cache.size(2), k_cache.size(0), slots.data_ptr(), contexts, int(width), heads, dim,
        float(scale), out.data_ptr(), _dtype(q), _stream(q))
    _lib.check(status, "prefill attention")
    return out


def prefill_supported(dtype: torch.dtype, head_dim: int) -> bool:
    """Whether :func:`prefill_attention` covers this element type and head size: bf16 with head dim 128, 256 or 512."""
    return dtype == torch.bfloat16 and head_dim in (128, 256, 512)


def splits_for(rows: int, heads: int, keys: int, block: int = 64, programs: int = 264) -> tuple[int, int]:
    """Key splits (a power of two, about ``programs`` programs in all) and the keys each split covers -- the
    reference's rule for its Triton launches (src/omniasr_trt/kernels.py:393-400), kept for callers that use it;
    the HIP launches choose their split with :func:`verify_chunk`."""
    want = max(1, programs // (rows * heads))
    splits = 1
    while splits * 2 <= want and splits * 2 * block <= keys:
        splits *= 2
    chunk = -(-keys // splits)
    return splits, -(-chunk // block) * block


def verify_chunk(rows: int, tokens: int, heads: int, head_dim: int, keys: int) -> int:
    """Keys per split of the verify attention at this launch shape (``omni_verify_attention_chunk``)."""
    return int(_lib.load().omni_verify_attention_chunk(rows, tokens, heads, head_dim, keys))


def _reach(reach) -> ctypes.Array:
    flat = [int(x) for pair in reach for x in pair]
    _need(len(flat) == 8, "reach: four (distance, tokens) pairs")
    return (ctypes.c_int32 * 8)(*flat)


def _propose_args(out, draft, draft_len, last, first, nxt, start, tokens, ngram, behind, ahead, reach, self_window,
                  self_min):
    _need(out.dtype == torch.int32 and out.stride(1) == 1, "out: [>=B, S] int32")
    _need(draft.dtype == torch.int32 and draft.stride(1) == 1, "draft: [>=B, C] int32")
    for name, t in (("draft_len", draft_len), ("last", last), ("first", first), ("next", nxt), ("start", start)):
        _index(t, name)
    width = next_power_of_2(behind + ahead + 1)  # the reference's anchor lanes (kernels.py:375)
    self_width = next_power_of_2(self_window)
    return [out.data_ptr(), out.stride(0), out.size(1), draft.data_ptr(), draft.stride(0), draft.size(1),
            draft_len.data_ptr(), last.data_ptr(), first.data_ptr(), nxt.data_ptr()], \
        [tokens, ngram, behind, ahead, width, self_width, self_min, _reach(reach)]


def propose(out: torch.Tensor, draft: torch.Tensor, draft_len: torch.Tensor, last: torch.Tensor,
            first: torch.Tensor, nxt: torch.Tensor, start: torch.Tensor, tokens: int, ngram: int, behind: int,
            ahead: int, reach: tuple, self_window: int, self_min: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Drafted decoding's proposals of rows 0..B-1 (B = ``last.numel()``): ``tokens`` ids each [B, k] (int64) and
    whether they come from the draft [B] (else from the row's own tokens); ``start`` [B] gets the draft position of
    the first one.  ``out`` [>=B, S] int32 generated tokens by position, ``draft`` [>=B, C] int32; ``draft_len``,
    ``last``, ``first``, ``nxt`` [B] int64.  (src/omniasr_trt/kernels.py:361-377)"""
    lib = _lib.load()
    b = last.numel()
    head, tail = _propose_args(out, draft, draft_len, last, first, nxt, start, tokens, ngram, behind, ahead, reach,
                               self_window, self_min)
    prop = torch.empty(b, tokens, device=out.device, dtype=torch.long)
    use_draft = torch.empty(b, device=out.device, dtype=torch.bool)
    status = lib.omni_propose(*head, prop.data_ptr(), use_draft.data_ptr(), start.data_ptr(), b, *tail,
                              _stream(out))
    _lib.check(status, "propose")
    return prop, use_draft


def spec_prepare(out: torch.Tensor, draft: torch.Tensor, draft_len: torch.Tensor, last: torch.Tensor,
                 first: torch.Tensor, nxt: torch.Tensor, start: torch.Tensor, tok: torch.Tensor, done: torch.Tensor,
                 capacity: int, tokens: int, ngram: int, behind: int, ahead: int, reach: tuple, self_window: int,
                 self_min: int):
    """:func:`propose` and the drafted step's inputs in one launch (src/omniasr_trt/spec.py:85-95).  Returns the
    fed tokens [B, k+1] (the newest token, then the proposal), positions and cache rows [B*(k+1)], key counts [B]
    (0 for finished rows) and ``use_draft`` [B]; ``start`` is written as by :func:`propose`."""
    lib = _lib.load()
    b = last.numel()
    head, tail = _propose_args(out, draft, draft_len, last, first, nxt, start, tokens, ngram, behind, ahead, reach,
                               self_window, self_min)
    _index(tok, "tok")
    _need(done.dtype == torch.bool and done.is_contiguous(), "done: bool [B]")
    width = tokens + 1
    dev = out.device
    fed = torch.empty(b, width, device=dev, dtype=torch.long)
    pos = torch.empty(b * width, device=dev, dtype=torch.long)
    slots = torch.empty(b * width, device=dev, dtype=torch.long)
    lengths = torch.empty(b, device=dev, dtype=torch.long)
    use_draft = torch.empty(b, device=dev, dtype=torch.bool)
    status = lib.omni_spec_prepare(*head, None, use_draft.data_ptr(), start.data_ptr(), b, *tail, tok.data_ptr(),
                                   done.data_ptr(), int(capacity), fed.data_ptr(), pos.data_ptr(), slots.data_ptr(),
                                   lengths.data_ptr(), _stream(out))
    _lib.check(status, "spec_prepare")
    return fed, pos, slots, lengths, use_draft


def _state_args(out, tok, last, done, draft_next, start, use_draft):
    _need(out.dtype == torch.int32 and out.stride(1) == 1, "out: [>=B, S] int32")
    for name, t in (("tok", tok), ("last", last)):
        _index(t, name)
    _need(done.dtype == torch.bool and done.is_contiguous(), "done: bool [B]")
    if draft_next is not None:
        _index(draft_next, "draft_next")
        _index(start, "start")
        _need(use_draft.dtype == torch.bool and use_draft.is_contiguous(), "use_draft: bool [B]")
    return [out.data_ptr(), out.stride(0), out.size(1), tok.data_ptr(), last.data_ptr(), done.data_ptr(),
            _ptr(draft_next), _ptr(start), _ptr(use_draft)]


def accept(tokens: torch.Tensor, nxt: torch.Tensor, out: torch.Tensor, tok: torch.Tensor, last: torch.Tensor,
           done: torch.Tensor, draft_next: torch.Tensor, start: torch.Tensor, use_draft: torch.Tensor, limit: int,
           eos: int) -> None:
    """In place on rows 0..B-1 after a drafted step: ``tokens`` fed [B, T] (the newest token, then the proposal) and
    ``nxt`` the argmax after each [B, T] (int64); ``out`` [>=B, S] int32, ``tok``/``last``/``draft_next``/``start``
    [B] int64, ``done``/``use_draft`` [B] bool.  A running row keeps argmax 0..n (n: its leading proposed tokens
    equal to the argmax before them, or the first EOS / position >= ``limit`` among those) at positions
    ``last + 1 + j``.  (src/omniasr_trt/kernels.py:380-390)"""
    lib = _lib.load()
    b, width = tokens.shape
    _index(tokens, "tokens")
    _index(nxt, "nxt")
    state = _state_args(out, tok, last, done, draft_next, start, use_draft)
    status = lib.omni_accept(tokens.data_ptr(), nxt.data_ptr(), *state, b, width, int(limit), int(eos),
                             _stream(tokens))
    _lib.check(status, "accept")


def greedy_accept(logits: torch.Tensor, tokens: torch.Tensor, out: torch.Tensor, tok: torch.Tensor,
                  last: torch.Tensor, done: torch.Tensor, draft_next: torch.Tensor | None,
                  start: torch.Tensor | None, use_draft: torch.Tensor | None, limit: int, eos: int,
                  nxt: torch.Tensor | None = None) -> torch.Tensor:
    """``F.log_softmax(logits, -1).argmax(-1)`` of the verify logits [B*T, V] followed by :func:`accept`
    (src/omniasr_trt/spec.py:106-108): an argmax workgroup per row, then the acceptance.  Returns the argmaxes
    [B, T] (written into ``nxt`` when given).
    ``draft_next`` / ``start`` / ``use_draft`` None: the one-token step's update (src/omniasr_trt/decode.py:218-224)."""
    lib = _lib.load()
    b, width = tokens.shape
    _index(tokens, "tokens")
    _need(logits.dim() == 2 and logits.size(0) == b * width and logits.stride(1) == 1, "logits: [B*T, V]")
    if nxt is None:
        nxt = torch.empty(b, width, device=logits.device, dtype=torch.long)
    _index(nxt, "nxt")
    state = _state_args(out, tok, last, done, draft_next, start, use_draft)
    status = lib.omni_greedy_accept(logits.data_ptr(), logits.stride(0), logits.size(1), _dtype(logits),
                                    tokens.data_ptr(), nxt.data_ptr(), *state, b, width, int(limit), int(eos),
                                    _stream(logits))
    _lib.check(status, "greedy_accept")
    return nxt


def _flags(t: torch.Tensor, name: str) -> None:
    _need(t.dtype == torch.bool and t.is_contiguous() and t.is_cuda, f"{name}: contiguous bool on the GPU")


def beam_prepare(groups: int, beams: int, ctx: torch.Tensor, k_step: torch.Tensor, group_done: torch.Tensor,
                 ptr: torch.Tensor, pos: torch.Tensor, gen_pos: torch.Tensor, ctx_len: torch.Tensor,
                 gen_len: torch.Tensor) -> None:
    """The beam step's bookkeeping before its layers, in one launch (src/omniasr_trt/beam.py:127-145): for the rows
    of groups 0..groups-1, ``pos`` = ctx + k - 1, ``gen_pos`` = max(k - 1, 0), ``gen_len`` = k (0 in a finished
    group), ``ctx_len`` = ctx (0 when finished), and a live row's ``ptr[r, gen_pos]`` = r.  ``ctx`` / ``k_step`` /
    ``group_done`` [>=groups]; ``ptr`` [>=rows, G] int32; the outputs [>=rows] / [>=groups] int64."""
    lib = _lib.load()
    for name, t in (("ctx", ctx), ("k_step", k_step), ("pos", pos), ("gen_pos", gen_pos), ("ctx_len", ctx_len),
                    ("gen_len", gen_len)):
        _index(t, name)
    _flags(group_done, "group_done")
    rows = groups * beams
    _need(ptr.dtype == torch.int32 and ptr.dim() == 2 and ptr.stride(1) == 1 and ptr.size(0) >= rows,
          "ptr: [>=rows, G] int32")
    _need(min(ctx.numel(), k_step.numel(), group_done.numel(), ctx_len.numel()) >= groups
          and min(pos.numel(), gen_pos.numel(), gen_len.numel()) >= rows, "state sizes")
    status = lib.omni_beam_prepare(groups, beams, ctx.data_ptr(), k_step.data_ptr(), group_done.data_ptr(),
                                   ptr.data_ptr(), ptr.stride(0), ptr.size(1), pos.data_ptr(), gen_pos.data_ptr(),
                                   ctx_len.data_ptr(), gen_len.data_ptr(), _stream(ptr))
    _lib.check(status, "beam_prepare")


def beam_take_over(best: torch.Tensor, flat: torch.Tensor, vocab: int, ptr: torch.Tensor, hist: torch.Tensor,
                   ended: torch.Tensor, score: torch.Tensor, count: torch.Tensor, tok: torch.Tensor,
                   k_step: torch.Tensor, group_done: torch.Tensor, ctx: torch.Tensor, limit: int, eos: int,
                   pad: int) -> None:
    """The beam step's bookkeeping after the top-k (src/omniasr_trt/beam.py:159-187), in one launch: ``best`` /
    ``flat`` [S, N] are ``offers.view(S, N * vocab).topk(N)``'s values and indices; every row of groups 0..S-1 takes
    over its parent's ``ptr`` / ``hist`` rows, score, count and finished flag, extended by its chosen token; then
    the groups' ``k_step`` and ``group_done``.  In place; equal to the torch ops bit for bit."""
    lib = _lib.load()
    groups, beams = best.shape
    rows = groups * beams
    _need(flat.shape == best.shape and flat.dtype == torch.long and flat.is_contiguous(), "flat: [S, N] int64")
    _need(best.is_contiguous() and best.dtype == score.dtype and score.dtype in (torch.float32, torch.float64)
          and score.is_contiguous(), "best / score: fp32 or fp64, contiguous, the same type")
    for name, t in (("count", count), ("tok", tok), ("k_step", k_step), ("ctx", ctx)):
        _index(t, name)
    _flags(ended, "ended")
    _flags(group_done, "group_done")
    for name, t in (("ptr", ptr), ("hist", hist)):
        _need(t.dtype == torch.int32 and t.dim() == 2 and t.stride(1) == 1 and t.size(0) >= rows,
              f"{name}: [>=rows, G] int32")
    _need(min(ended.numel(), score.numel(), count.numel(), tok.numel()) >= rows
          and min(k_step.numel(), group_done.numel(), ctx.numel()) >= groups, "state sizes")
    status = lib.omni_beam_take_over(groups, beams, int(vocab), best.data_ptr(), flat.data_ptr(), ptr.data_ptr(),
                                     ptr.stride(0), ptr.size(1), hist.data_ptr(), hist.stride(0), hist.size(1),
                                     ended.data_ptr(), score.data_ptr(), score.element_size(), count.data_ptr(),
                                     tok.data_ptr(), k_step.data_ptr(), group_done.data_ptr(), ctx.data_ptr(),
                                     int(limit), int(eos), int(pad), _stream(best))
    _lib.check(status, "beam_take_over")


def beam_select_supported(logits: torch.Tensor, score: torch.Tensor, beams: int) -> bool:
    """Whether ``beam_select`` takes these logits: bf16 [rows, V] on the GPU (unit stride, 16-byte aligned rows, V a
    multiple of 8, at most 16384), fp32 scores, 1..16 beams."""
    return (logits.is_cuda and logits.dtype == torch.bfloat16 and logits.dim() == 2 and logits.stride(1) == 1
            and logits.stride(0) % 8 == 0 and logits.data_ptr() % 16 == 0 and logits.size(1) % 8 == 0
            and beams <= logits.size(1) <= 16384 and 1 <= beams <= 16 and score.dtype == torch.float32)


def beam_select(logits: torch.Tensor, score: torch.Tensor, count: torch.Tensor, ended: torch.Tensor, beams: int,
                length_norm: bool, eos: int, *, fused_log_softmax: bool = False,
                tickets: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """The beam step's choice (src/omniasr_trt/beam.py:162-175): ``F.log_softmax(logits)`` in bf16, the offers
    (score + logp; with ``length_norm``, once the group's row 0 has tokens, (score * count + logp) / (count + 1); a
    finished row offers only ``eos``, at its score) and ``offers.view(S, N * V).topk(N)`` -- returns (best [S, N]
    fp32, flat [S, N] int64), best first, equal values in the order of their flat index.  ``score`` / ``count`` /
    ``ended``: the rows' state (fp32 / int64 / bool, at least S * N rows).

    The log-softmax is torch's own (one launch), and the offers and top-k are one launch of ``omni_beam_select``:
    the choice is the one torch's ops make, bit for bit.  ``fused_log_softmax=True`` computes the log-softmax in the
    same launch instead, in the kernel's own summation order: a logp on a bf16 rounding boundary can then round the
    other way (measured: 3 of 12,472 group-steps of bf16 searches chose differently).  ``tickets``: int32, one per
    group, zero (left zero); by default a per-device buffer shared by every caller, so searches that run at once on
    two streams of one GPU each pass their own."""
    lib = _lib.load()
    _need(beam_select_supported(logits, score, beams), "beam_select: bf16 logits [S*N, V] (8 | V <= 16384, unit "
          "stride), fp32 score, 1..16 beams")
    rows, vocab = logits.shape
    _need(rows % beams == 0, "beam_select: rows a multiple of beams")
    _need(score.is_contiguous() and score.numel() >= rows, "score: fp32 [>= rows]")
    _index(count, "count")
    _flags(ended, "ended")
    _need(count.numel() >= rows and ended.numel() >= rows, "count / ended: [>= rows]")
    groups = rows // beams
    if tickets is None:
        tickets = _tickets(_select_tickets, logits.device, groups, "beam_select", 256)
    _need(tickets.is_cuda and tickets.dtype == torch.int32 and tickets.is_contiguous() and tickets.numel() >= groups
          and tickets.device == logits.device, "tickets: int32 [>= groups] on the logits' device")
    if fused_log_softmax:
        rows_in, kind = logits, _lib.SELECT_LOGITS
    else:
        rows_in, kind = F.log_softmax(logits, dim=-1), _lib.SELECT_LOGP  # torch's own rounding: the reference's logp
    best = torch.empty(groups, beams, device=logits.device, dtype=torch.float32)
    flat = torch.empty(groups, beams, device=logits.device, dtype=torch.long)
    ws = lib.omni_beam_select_workspace(groups, beams)
    workspace = torch.empty(max(ws, 256), device=logits.device, dtype=torch.uint8)
    status = lib.omni_beam_select(rows_in.data_ptr(), rows_in.stride(0), groups, beams, vocab, score.data_ptr(),
                                  count.data_ptr(), ended.data_ptr(), int(bool(length_norm)), int(eos),
                                  best.data_ptr(), flat.data_ptr(), workspace.data_ptr(), workspace.numel(),
                                  tickets.data_ptr(), kind, _lib.BF16, _stream(logits))
    _lib.check(status, "beam_select")
    return best, flat


def layer_ops_supported(x: torch.Tensor) -> bool:
    """Whether ``rms_norm`` (x [N, D], D <= 8192) / ``silu_mul`` (x [N, 2F]) take this activation: bf16 rows on the
    GPU, 16-byte aligned, the row length a multiple of 16 (of 8 for each half)."""
    return (x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 2 and x.stride(1) == 1 and x.stride(0) % 8 == 0
            and x.size(1) % 16 == 0 and x.data_ptr() % 16 == 0)


def rms_norm_supported(x: torch.Tensor, weight: torch.Tensor) -> bool:
    return (layer_ops_supported(x) and x.size(1) <= 8192 and weight.dtype == x.dtype and weight.is_contiguous()
            and weight.numel() == x.size(1) and weight.data_ptr() % 16 == 0)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``F.rms_norm(x, (D,), weight, eps)`` for bf16 x [N, D] (D <= 8192, a multiple of 8): fp32 arithmetic, one
    rounding after both products.  The norm of the reference's decoder layers (RMSNorm in
    src/omniasr_trt/modeling.py, run by SpecDecoder.step, spec.py:97-106)."""
    lib = _lib.load()
    _need(rms_norm_supported(x, weight), "rms_norm: bf16 x [N, D <= 8192] (16 | D, unit stride) and weight [D]")
    y = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    status = lib.omni_rms_norm(x.data_ptr(), x.stride(0), weight.data_ptr(), y.data_ptr(), y.stride(0), x.size(0),
                               x.size(1), float(eps), _lib.BF16, _stream(x))
    _lib.check(status, "rms_norm")
    return y


def silu_mul(gate_inner: torch.Tensor) -> torch.Tensor:
    """``inner * F.silu(gate)`` for ``gate, inner = gate_inner.chunk(2, -1)``, bf16 [N, 2F] -> [N, F]: silu(gate)
    rounded to bf16, then the product, as torch's two kernels round.  The FFN of the reference's decoder layers
    (spec.py:97-106 over the fused gate|inner projection of decode.py:34-54)."""
    lib = _lib.load()
    _need(layer_ops_supported(gate_inner), "silu_mul: bf16 gate_inner [N, 2F] with F a multiple of 8")
    f = gate_inner.size(1) // 2
    out = torch.empty(gate_inner.size(0), f, device=gate_inner.device, dtype=gate_inner.dtype)
    status = lib.omni_silu_mul(gate_inner.data_ptr(), gate_inner.stride(0), out.data_ptr(), out.stride(0),
                               gate_inner.size(0), f, _lib.BF16, _stream(gate_inner))
    _lib.check(status, "silu_mul")
    return out

"""numpy restatement of the verify step's kernels (test infrastructure; see oracle/__init__.py).

Arrays: token buffers int32 / int64 as the reference's; bf16 tensors are float32 arrays of bf16-exact
values and every result that the reference stores in bf16 is rounded with :func:`oracle.bf16.round_to`.
"""

from __future__ import annotations

import numpy as np

from .bf16 import round_to

F32 = np.float32


# ---------------------------------------------------------------------------------------------- RoPE + append

def rope_kv(qkv: np.ndarray, cs: np.ndarray, pos: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, heads: int,
            slots: np.ndarray | None = None, cache_pos: np.ndarray | None = None, dtype: str = "bf16") -> np.ndarray:
    """Rotated q [N, H, D]; k (rotated) and v written in place at (slots[n], h, cache_pos[n]).

    Rotation of ``apply_rope`` (src/omniasr_trt/modeling.py:301-306): interleaved pairs (re, im) at position p
    become (re*c - im*s, re*s + im*c) with (c, s) = cs[p, j]; numpy evaluates each float32 product and the
    difference / sum with their own rounding, as PyTorch's element-wise kernels do; then the result is rounded
    to the element type.  Indexing of ``_rope_kv`` (src/omniasr_trt/kernels.py:31-54): cache row ``slots[n]``
    (default n), position ``cache_pos[n]`` (default ``pos[n]``).
    Pinned by: the closed form (a rotation preserves each pair's norm and composes additively in the angle; a
    zero angle is the identity), the V copy being exact, and index invariants (tests/test_oracle.py)."""
    n = qkv.shape[0]
    d = qkv.shape[1] // (3 * heads)
    x = np.asarray(qkv, dtype=F32).reshape(n, 3, heads, d // 2, 2)
    t = np.asarray(cs, dtype=F32)[np.asarray(pos)]  # [n, d/2, 2]
    c, s = t[:, None, None, :, 0], t[:, None, None, :, 1]
    re, im = x[..., 0], x[..., 1]
    out_re = (re * c) - (im * s)
    out_im = (re * s) + (im * c)
    rot = np.stack([out_re, out_im], -1).reshape(n, 3, heads, d).astype(F32)
    q = round_to(rot[:, 0], dtype)
    k = round_to(rot[:, 1], dtype)
    v = np.asarray(qkv, dtype=F32).reshape(n, 3, heads, d)[:, 2]
    rows = np.arange(n) if slots is None else np.asarray(slots)
    cp = np.asarray(pos) if cache_pos is None else np.asarray(cache_pos)
    for i in range(n):  # in token order: a later token to the same place wins (the kernels leave that undefined)
        k_cache[rows[i], :, cp[i]] = k[i]
        v_cache[rows[i], :, cp[i]] = v[i]
    return q


def rope_table(head_dim: int, positions: int, theta: float = 10_000.0) -> np.ndarray:
    """cos/sin [positions, head_dim/2, 2] in float64 from the closed form p * theta^(-2j/head_dim)
    (src/omniasr_trt/modeling.py:293-298) -- to check the product's fp32 table, not to replace it."""
    inv = 1.0 / theta ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim)
    ang = np.outer(np.arange(positions, dtype=np.float64), inv)
    return np.stack([np.cos(ang), np.sin(ang)], -1)


# ---------------------------------------------------------------------------------------------- attention

def verify_attention(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, lengths: np.ndarray, tokens: int,
                     scale: float) -> np.ndarray:
    """Causal multi-query attention in float64: query i of row b (q row b*tokens + i) over keys
    [0, lengths[b] + i) of cache row b; an empty range gives zeros.  (src/omniasr_trt/kernels.py:56-113 with
    CAUSAL=True, 146-161; the T = 1 case is kernels.py:163-211.)  Pinned by: the textbook formula on tiny inputs
    against a per-query loop, the log-sum-exp merge identity, and the empty-range rule (tests/test_oracle.py)."""
    rows_total, heads, d = q.shape
    b_rows = rows_total // tokens
    out = np.zeros((rows_total, heads, d), dtype=np.float64)
    cap = k_cache.shape[2]
    for b in range(b_rows):
        n = int(min(max(int(lengths[b]), 0), cap))
        total = min(n + tokens - 1, cap)
        if total <= 0:
            continue
        k = np.asarray(k_cache[b, :, :total], dtype=np.float64)  # [H, L, D]
        v = np.asarray(v_cache[b, :, :total], dtype=np.float64)
        qb = np.asarray(q[b * tokens:(b + 1) * tokens], dtype=np.float64)  # [T, H, D]
        sc = np.einsum("thd,hld->thl", qb, k, optimize=True) * scale  # [T, H, L]
        j = np.arange(total)
        visible = j[None, :] < (n + np.arange(tokens))[:, None]  # [T, L]
        sc = np.where(visible[:, None, :], sc, -np.inf)
        top = sc.max(-1, keepdims=True)
        top = np.where(np.isfinite(top), top, 0.0)
        w = np.exp(sc - top)
        den = w.sum(-1, keepdims=True)
        o = np.einsum("thl,hld->thd", w, v, optimize=True) / np.where(den > 0, den, 1.0)
        out[b * tokens:(b + 1) * tokens] = o
    return out


def beam_attention(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, ctx_len: np.ndarray, kg: np.ndarray,
                   vg: np.ndarray, ptr: np.ndarray, gen_len: np.ndarray, beams: int, scale: float) -> np.ndarray:
    """Beam attention in float64: row r = g*beams + i over the first ctx_len[g] keys of context row g, then its
    generated keys j < gen_len[r], key j taken from row ptr[r, j] of kg / vg; no key at all gives zeros.
    (src/omniasr_trt/kernels.py:309-332: ``_beam_ctx`` with CAUSAL=False, ``_beam_gen``, ``_beam_combine``.)
    Pinned by: one beam with no generated keys is verify_attention at T = 1; context-free rows whose pointers all
    name the row itself are verify_attention over that row of kg; a gather-then-softmax restatement on small
    inputs (tests/test_oracle.py)."""
    rows, heads, d = q.shape
    out = np.zeros((rows, heads, d), dtype=np.float64)
    for r in range(rows):
        g = r // beams
        nc = int(min(max(int(ctx_len[g]), 0), kc.shape[2]))
        ng = int(min(max(int(gen_len[r]), 0), kg.shape[2]))
        if nc + ng == 0:
            continue
        j = np.arange(ng)
        src = np.clip(np.asarray(ptr[r, :ng], dtype=np.int64), 0, kg.shape[0] - 1)
        k = np.concatenate([np.asarray(kc[g, :, :nc], dtype=np.float64),
                            np.asarray(kg[src, :, j], dtype=np.float64).transpose(1, 0, 2)], 1)  # [H, L, D]
        v = np.concatenate([np.asarray(vc[g, :, :nc], dtype=np.float64),
                            np.asarray(vg[src, :, j], dtype=np.float64).transpose(1, 0, 2)], 1)
        sc = np.einsum("hd,hld->hl", np.asarray(q[r], dtype=np.float64), k, optimize=True) * scale
        w = np.exp(sc - sc.max(-1, keepdims=True))
        out[r] = np.einsum("hl,hld->hd", w, v, optimize=True) / w.sum(-1, keepdims=True)
    return out


# ---------------------------------------------------------------------------------------------- beam step

def beam_prepare(groups: int, beams: int, ctx, k_step, group_done, ptr):
    """The beam step before its layers (src/omniasr_trt/beam.py:133-145), row by row: returns (pos, gen_pos, ctx_len,
    gen_len) and writes a live row's own index at ptr[r, gen_pos[r]] in place.
    Pinned by: a hand-computed case and the reference's vectorised formulation of the same step
    (tests/test_oracle.py)."""
    rows = groups * beams
    pos = np.zeros(rows, np.int64)
    gen_pos = np.zeros(rows, np.int64)
    gen_len = np.zeros(rows, np.int64)
    ctx_len = np.zeros(groups, np.int64)
    for g in range(groups):
        done = bool(group_done[g])
        ctx_len[g] = 0 if done else ctx[g]
        for i in range(beams):
            r = g * beams + i
            k = int(k_step[g])
            pos[r] = ctx[g] - 1 + k
            gen_pos[r] = max(k - 1, 0)
            gen_len[r] = 0 if done else k
            if not done and gen_pos[r] < ptr.shape[1]:
                ptr[r, gen_pos[r]] = r
    return pos, gen_pos, ctx_len, gen_len


def beam_take_over(best, flat, vocab: int, ptr, hist, ended, score, count, tok, k_step, group_done, ctx, limit: int,
                   eos: int, pad: int) -> None:
    """The beam step after the per-group top-N (src/omniasr_trt/beam.py:170-187), row by row, in place: each row of a
    live group takes over its parent's pointers, history, score, token count and finished flag, extended by its
    chosen token (EOS after a finished parent); then the group's step counter and finished flag.
    Pinned by: a hand-computed case, invariants (a finished group keeps its state; rows are a permutation of the old
    ones within their group) and the reference's vectorised formulation (tests/test_oracle.py)."""
    groups, beams = best.shape
    old_ptr, old_hist = ptr.copy(), hist.copy()
    old_ended, old_score, old_count, old_tok = ended.copy(), score.copy(), count.copy(), tok.copy()
    for g in range(groups):
        live = not bool(group_done[g])
        k = int(k_step[g])
        for i in range(beams):
            r = g * beams + i
            p = g * beams + int(flat[g, i]) // vocab if live else r
            chosen = int(flat[g, i]) % vocab if live else int(old_tok[r])
            if old_ended[p]:
                chosen = eos
            ptr[r] = old_ptr[p]
            hist[r] = old_hist[p]
            if live and k < hist.shape[1]:
                hist[r, k] = chosen
            extends = live and not old_ended[p]
            score[r] = best[g, i] if extends else old_score[p]
            count[r] = old_count[p] + (1 if extends and chosen not in (pad, eos) else 0)
            ended[r] = (chosen == eos) if live else old_ended[p]
            tok[r] = chosen
        k_step[g] = k + (1 if live else 0)
        rows = slice(g * beams, (g + 1) * beams)
        group_done[g] = bool(group_done[g]) or bool(np.all(ended[rows])) or ctx[g] - 1 + k_step[g] - 1 >= limit


# ---------------------------------------------------------------------------------------------- argmax

def log_softmax_f32(logits: np.ndarray, lse_shift: int = 0) -> np.ndarray:
    """The float32 log-probabilities before the store's rounding, in the order of PyTorch's GPU kernel
    (``LogSoftMaxForwardEpilogue``: ``input - max_input - logsum``, max and sum kept in float32): m = max,
    lse = log(sum exp(x - m)), y = (x - m) - lse.  ``lse_shift`` moves lse by that many float32 ulps."""
    x = np.asarray(logits, dtype=F32)
    m = x.max(-1, keepdims=True)
    s = np.exp((x - m).astype(F32)).astype(F32).sum(-1, keepdims=True, dtype=np.float64).astype(F32)
    lse = np.log(s).astype(F32)
    for _ in range(abs(lse_shift)):
        lse = np.nextafter(lse, np.float32(np.inf) if lse_shift > 0 else np.float32(-np.inf)).astype(F32)
    return ((x - m).astype(F32) - lse).astype(F32)


def log_softmax_argmax(logits: np.ndarray, dtype: str = "bf16", lse_shift: int = 0) -> np.ndarray:
    """``F.log_softmax(logits, -1).argmax(-1)`` (src/omniasr_trt/spec.py:107) as PyTorch evaluates it on the GPU:
    :func:`log_softmax_f32` rounded to the logits' type, then the first index of the maximum.  ``lse_shift``: see
    :func:`log_softmax_f32` (finds rows whose result depends on the last bits of lse, i.e. on the summation
    order).  Pinned by: PyTorch's float32 ``F.log_softmax`` (CPU) elementwise to a few ulps and its argmax after
    rounding, PyTorch's own GPU op in the GPU tests, and planted known answers (tests/test_oracle.py).  PyTorch's
    CPU kernel for bf16 input is not the reference: it rounds the sum and its log to bf16 first."""
    y = round_to(log_softmax_f32(logits, lse_shift), dtype)
    return y.argmax(-1).astype(np.int64)


def argmax_is_fragile(logits: np.ndarray, dtype: str = "bf16", ulps: int = 4) -> np.ndarray:
    """Rows whose argmax changes when lse moves by up to ``ulps`` float32 ulps either way: their result depends on
    how the exponentials are summed, which no two implementations share bit for bit."""
    base = log_softmax_argmax(logits, dtype)
    fragile = np.zeros(base.shape, dtype=bool)
    for sh in range(1, ulps + 1):
        fragile |= log_softmax_argmax(logits, dtype, sh) != base
        fragile |= log_softmax_argmax(logits, dtype, -sh) != base
    return fragile


# ---------------------------------------------------------------------------------------------- accept

def accept(tokens, nxt, out, tok, last, done, draft_next, start, use_draft, limit: int, eos: int) -> None:
    """In place, rows with done == 0 (src/omniasr_trt/kernels.py:271-291): p = last + 1; kept = leading j with
    tokens[j+1] == nxt[j] (at most T-1); stop_j = (nxt[j] == eos or p + j >= limit) and j <= kept; n = first stop
    or kept; out[min(p+j, S-1)] = nxt[j] for j <= n; tok = nxt[n]; last = p + n; done = any stop; draft_next =
    (use_draft ? start : draft_next) + n + 1 (when draft_next is given).  Pinned by: the one-token reduction to
    the greedy update (src/omniasr_trt/decode.py:219-224, :func:`greedy_update`), hand-computed known answers and
    golden vectors of the reference's own kernel (tests/golden)."""
    b_rows, width = tokens.shape
    cap = out.shape[1]
    for b in range(b_rows):
        if done[b]:
            continue
        p = int(last[b]) + 1
        g = [int(x) for x in nxt[b]]
        kept = width - 1
        for j in range(width - 1):
            if int(tokens[b, j + 1]) != g[j]:
                kept = j
                break
        stops = [j for j in range(kept + 1) if g[j] == eos or p + j >= limit]
        n = stops[0] if stops else kept
        for j in range(n + 1):
            out[b, min(p + j, cap - 1)] = g[j]
        tok[b] = g[n]
        last[b] = p + n
        done[b] = bool(stops)
        if draft_next is not None:
            draft_next[b] = (int(start[b]) if use_draft[b] else int(draft_next[b])) + n + 1


def greedy_update(nxt, out, tok, last, done, limit: int, eos: int) -> None:
    """The one-token step's update in PyTorch order (src/omniasr_trt/decode.py:219-224): p = last + running;
    out[p] = running ? nxt : out[p]; done |= running and (nxt == eos or p >= limit); tok = running ? nxt : tok;
    last = p."""
    running = ~done.astype(bool)
    p = last + running.astype(np.int64)
    rows = np.arange(len(p))
    kept = out[rows, p]
    out[rows, p] = np.where(running, nxt.astype(out.dtype), kept)
    done |= running & ((nxt == eos) | (p >= limit))
    tok[:] = np.where(running, nxt, tok)
    last[:] = p


# ---------------------------------------------------------------------------------------------- propose

def need_for(dist: np.ndarray, reach, ngram: int) -> np.ndarray:
    need = np.full(np.shape(dist), ngram, dtype=np.int64)
    for r, n in reversed(list(reach)):
        need = np.where(dist <= r, n, need)
    return need


def _leading_matches(source: np.ndarray, at: np.ndarray, live: np.ndarray, hist: np.ndarray,
                     hist_ok: np.ndarray) -> np.ndarray:
    """For each candidate position ``at`` [W]: the number of leading t with source[at - t] == hist[t]."""
    ngram = len(hist)
    score = np.zeros(at.shape, dtype=np.int64)
    alive = live.copy()
    for t in range(ngram):
        a = at - t
        alive &= (a >= 0) & bool(hist_ok[t]) & (a < len(source))
        vals = np.where(alive, source[np.clip(a, 0, len(source) - 1)], -2)
        alive &= vals == hist[t]
        score += alive
    return score


def propose(out, draft, draft_len, last, first, nxt, k: int, ngram: int, behind: int, ahead: int, reach,
            anchor_width: int, self_width: int, self_min: int):
    """Proposals [B, k] int64, use_draft [B] bool, start [B] int64 of ``_propose`` (src/omniasr_trt/kernels.py:
    214-268; anchor lanes ``anchor_width = pow2(behind + ahead + 1)``, own lanes ``self_width =
    pow2(self_window)``, kernels.py:375).  Pinned by: golden vectors of the reference's ``reference_propose``
    (tests/golden/propose_*.npz), the loop restatement :func:`propose_loops` on tiny inputs, and invariants
    (a perfect draft proposes its next tokens; a repetition loop continues periodically)."""
    b_rows = len(last)
    prop = np.zeros((b_rows, k), dtype=np.int64)
    use = np.zeros(b_rows, dtype=bool)
    start = np.zeros(b_rows, dtype=np.int64)
    for b in range(b_rows):
        lst, fst, nx, dl = int(last[b]), int(first[b]), int(nxt[b]), int(draft_len[b])
        orow, drow = np.asarray(out[b]), np.asarray(draft[b])
        t = np.arange(ngram)
        hp = lst - t
        hist_ok = hp >= fst
        hist = np.where(hist_ok & (hp >= 0) & (hp < len(orow)), orow[np.clip(hp, 0, len(orow) - 1)], -1)
        i = np.arange(anchor_width)
        off = i - behind
        anchor = nx - 1 + off
        live = (off <= ahead) & (anchor < dl)
        score = _leading_matches(drow, anchor, live, hist, hist_ok)
        dist = np.abs(off)
        rank = np.where((score >= need_for(dist, reach, ngram)) & (off <= ahead), score * 256 - dist, -1)
        best = int(np.argmax(rank))  # first maximum
        found = rank[best] >= 0
        drafted = int(score[best]) if found else 0
        st = nx + best - behind if found else nx
        back = lst - 1 - np.arange(self_width)
        sscore = _leading_matches(orow, back, back >= fst, hist, hist_ok)
        jj = int(np.argmax(sscore))
        mine = int(sscore[jj])
        j = lst - 1 - jj
        period = max(lst - j, 1)
        ud = mine < self_min or mine <= drafted
        for q in range(k):
            if ud:
                at = st + q
                prop[b, q] = drow[at] if 0 <= at < dl and at < len(drow) else 0
            else:
                at = j + 1 + q % period
                prop[b, q] = orow[at] if 0 <= at < len(orow) else 0
        use[b], start[b] = ud, st
    return prop, use, start


def propose_loops(out, draft, draft_len, last, first, nxt, k, ngram, behind, ahead, reach, anchor_width,
                  self_width, self_min):
    """:func:`propose` written as plain loops over candidates, comparing token lists -- the brute-force check on
    tiny inputs."""
    res_prop, res_use, res_start = [], [], []
    for b in range(len(last)):
        lst, fst, nx, dl = int(last[b]), int(first[b]), int(nxt[b]), int(draft_len[b])
        orow = [int(x) for x in out[b]]
        drow = [int(x) for x in draft[b]]
        newest = []  # h_0, h_1, ... while valid
        for t in range(ngram):
            if lst - t < fst:
                break
            newest.append(orow[lst - t] if 0 <= lst - t < len(orow) else -1)

        def run(seq, end, limit_len):
            count = 0
            for t, h in enumerate(newest):
                pos_ = end - t
                if pos_ < 0 or pos_ >= limit_len or seq[pos_] != h:
                    break
                count += 1
            return count

        best_rank, best_i, best_score = -2, 0, 0  # below every rank: the first anchor sets it
        for i in range(anchor_width):
            off = i - behind
            anchor = nx - 1 + off
            score = run(drow, anchor, min(len(drow), dl)) if (off <= ahead and anchor < dl) else 0
            need = ngram
            for r, nn in reach:
                if abs(off) <= r:
                    need = nn
                    break
            rank = score * 256 - abs(off) if (score >= need and off <= ahead) else -1
            if rank > best_rank:  # strictly greater: the first of equal ranks stays
                best_rank, best_i, best_score = rank, i, score
        found = best_rank >= 0
        drafted = best_score if found else 0
        st = nx + best_i - behind if found else nx
        mine, jj = -1, 0
        for i in range(self_width):
            back = lst - 1 - i
            score = run(orow, back, len(orow)) if back >= fst else 0
            if score > mine:
                mine, jj = score, i
        j = lst - 1 - jj
        period = max(lst - j, 1)
        ud = mine < self_min or mine <= drafted
        props = []
        for q in range(k):
            if ud:
                at = st + q
                props.append(drow[at] if 0 <= at < dl and at < len(drow) else 0)
            else:
                at = j + 1 + q % period
                props.append(orow[at] if 0 <= at < len(orow) else 0)
        res_prop.append(props)
        res_use.append(ud)
        res_start.append(st)
    return np.array(res_prop, dtype=np.int64), np.array(res_use), np.array(res_start, dtype=np.int64)


def spec_prepare(out, draft, draft_len, last, first, nxt, tok, done, capacity: int, k: int, ngram, behind, ahead,
                 reach, anchor_width, self_width, self_min):
    """Proposal plus the drafted step's inputs (src/omniasr_trt/spec.py:85-95): tokens [B, k+1] = (tok, proposal);
    pos = min(running ? p + j : last, capacity - 1) with p = last + running; slots = row; lengths = running ?
    p + 1 : 0."""
    prop, use, start = propose(out, draft, draft_len, last, first, nxt, k, ngram, behind, ahead, reach,
                               anchor_width, self_width, self_min)
    b_rows = len(last)
    width = k + 1
    running = ~np.asarray(done, dtype=bool)
    p = np.asarray(last) + running.astype(np.int64)
    tokens = np.concatenate([np.asarray(tok, dtype=np.int64)[:, None], prop], 1)
    j = np.arange(width)
    pos = np.where(running[:, None], p[:, None] + j, np.asarray(last)[:, None])
    pos = np.minimum(pos, capacity - 1).reshape(-1)
    slots = np.repeat(np.arange(b_rows), width)
    lengths = np.where(running, p + 1, 0)
    return tokens, pos, slots, lengths, use, start


# ---------------------------------------------------------------------------------------------- drafts

def frames_to_draft(frames, segment: int, segment_samples: int, hop: int = 320, margin=(25, 50), eos: int = 2):
    """Segment ``segment``'s draft from CTC frame argmaxes (src/omniasr_trt/llm.py:74-85), as a loop: frames
    [lo - margin0, hi + margin1) with lo, hi the segment's frame range; a frame is kept when it differs from the
    frame before it (within that window) and is > eos; ``before`` counts the kept frames before lo."""
    lo, hi = segment * segment_samples // hop, (segment + 1) * segment_samples // hop
    begin = max(0, lo - margin[0])
    window = [int(x) for x in frames[begin: hi + margin[1]]]
    ids, before = [], 0
    for i, f in enumerate(window):
        if (i == 0 or f != window[i - 1]) and f > eos:
            ids.append(f)
            if begin + i < lo:
                before += 1
    return ids, before

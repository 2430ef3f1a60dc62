"""The oracle pinned before it is trusted (CPU): golden vectors of the reference's own kernels, PyTorch's own ops on
the same inputs, closed forms, invariants and brute force on tiny inputs."""

from pathlib import Path

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import bf16
from oracle import reference as oref
from oracle import verify as ov

GOLD = Path(__file__).parent / "golden"
NGRAM, BEHIND, AHEAD, SELF_WINDOW, SELF_MIN = 8, 64, 160, 256, 3
REACH = ((1, 1), (4, 2), (12, 4), (40, 6))
W, SW = 256, 256  # pow2(BEHIND + AHEAD + 1), pow2(SELF_WINDOW)


def _bf16_np(t: torch.Tensor) -> np.ndarray:
    return t.float().numpy()


# ---------------------------------------------------------------------------------------------- bf16

def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(200_000) * 10.0 ** rng.integers(-38, 38, 200_000)).astype(np.float32)
    # exact ties (low half 0x8000) with even and odd upper halves, and the edges
    ties = (np.arange(0x3F80, 0x3F80 + 512, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    edges = np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1e-40, -1e-40, 1.17e-38], dtype=np.float32)
    x = np.concatenate([x, ties, edges])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bf16.to_bits(x), want)
    assert bf16.to_bits(np.array([np.nan], dtype=np.float32))[0] == 0x7FC0


# ---------------------------------------------------------------------------------------------- RoPE

@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_rope_oracle_is_pytorchs_rounding(dtype):
    """numpy's float32 evaluation order equals PyTorch's element-wise ``apply_rope`` bit for bit."""
    g = torch.Generator().manual_seed(1)
    n, h, d = 7, 4, 128
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    qkv = torch.randn(n, 3 * h * d, generator=g).to(tdt)
    cs = oref.rope_table(d, 4096)
    pos = torch.tensor([0, 1, 17, 999, 4095, 2048, 3])
    kc = np.zeros((n, h, 4096, d), np.float32)
    vc = np.zeros_like(kc)
    q = ov.rope_kv(_bf16_np(qkv), cs.numpy(), pos.numpy(), kc, vc, h, dtype=dtype)
    rq, rk, rv = qkv.view(n, 3, h, d).unbind(1)
    c = cs[pos][:, None]
    np.testing.assert_array_equal(q, oref.apply_rope(rq, c).float().numpy())
    rows = np.arange(n)
    np.testing.assert_array_equal(kc[rows, :, pos.numpy()], oref.apply_rope(rk, c).float().numpy())
    np.testing.assert_array_equal(vc[rows, :, pos.numpy()], rv.float().numpy())


def test_rope_table_closed_form():
    """The product's fp32 table is the standard RoPE table: (cos, sin) of p * theta^(-2j/D), pairs interleaved."""
    from omniasr_trt_amd import modeling

    for d in (16, 128, 512):
        cfg = modeling.DecoderConfig(model_dim=d * 2, num_heads=2)
        t = modeling.rope_table(cfg).numpy().astype(np.float64)
        ref = ov.rope_table(d, cfg.max_seq_len)
        # fp32 angles p * inv lose up to ~p * 2^-24 rad: the bound grows with the position
        err = np.abs(t - ref).max(axis=(1, 2))
        bound = 1e-6 + np.arange(cfg.max_seq_len) * 2.0 ** -22
        assert (err <= bound).all()
        assert np.array_equal(t[0, :, 0], np.ones(d // 2)) and np.array_equal(t[0, :, 1], np.zeros(d // 2))


def test_rope_rotation_properties():
    """A rotation keeps each pair's norm, position 0 is the identity, and k/v land at (slot, head, position)."""
    rng = np.random.default_rng(3)
    n, h, d, s = 6, 3, 16, 40
    qkv = rng.standard_normal((n, 3 * h * d)).astype(np.float32)
    cs = ov.rope_table(d, s).astype(np.float32)
    pos = np.array([0, 5, 39, 7, 0, 12])
    slots = np.array([2, 0, 1, 2, 3, 1])
    cache_pos = np.array([1, 2, 3, 4, 5, 6])
    kc = np.full((4, h, s, d), 7.0, np.float32)
    vc = np.full_like(kc, 7.0)
    q = ov.rope_kv(qkv, cs, pos, kc, vc, h, slots, cache_pos, dtype="f32")
    x = qkv.reshape(n, 3, h, d // 2, 2)
    np.testing.assert_allclose(np.linalg.norm(q.reshape(n, h, d // 2, 2), axis=-1), np.linalg.norm(x[:, 0], axis=-1),
                               rtol=1e-5)
    np.testing.assert_array_equal(q[0], qkv.reshape(n, 3, h, d)[0, 0])  # angle 0
    for i in range(n):
        np.testing.assert_array_equal(vc[slots[i], :, cache_pos[i]], qkv.reshape(n, 3, h, d)[i, 2])
    touched = np.zeros(kc.shape[:3], bool)
    touched[slots, :, cache_pos] = True
    assert (kc[~touched] == 7.0).all() and (vc[~touched] == 7.0).all()
    # rotating by p then by r equals rotating by p + r (fp64 closed form)
    t64 = ov.rope_table(d, 64)
    a = x[1, 0].astype(np.float64)
    z = a[..., 0] + 1j * a[..., 1]
    rot = lambda z, p: z * (t64[p, :, 0] + 1j * t64[p, :, 1])  # noqa: E731
    np.testing.assert_allclose(rot(rot(z, 5), 7), rot(z, 12), rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------------------------- attention

def test_attention_oracle_is_the_textbook_formula():
    rng = np.random.default_rng(4)
    b, h, d, t, cap = 3, 2, 8, 4, 12
    q = rng.standard_normal((b * t, h, d))
    kc = rng.standard_normal((b + 1, h, cap, d))
    vc = rng.standard_normal((b + 1, h, cap, d))
    lengths = np.array([5, 0, 1])
    out = ov.verify_attention(q, kc, vc, lengths, t, 0.3)
    for r in range(b):
        for i in range(t):
            n = lengths[r] + i
            for hh in range(h):
                if n == 0:
                    assert np.all(out[r * t + i, hh] == 0)
                    continue
                s = [0.3 * sum(q[r * t + i, hh, e] * kc[r, hh, j, e] for e in range(d)) for j in range(n)]
                mx = max(s)
                w = [math.exp(x - mx) for x in s]
                o = [sum(w[j] * vc[r, hh, j, e] for j in range(n)) / sum(w) for e in range(d)]
                np.testing.assert_allclose(out[r * t + i, hh], o, rtol=1e-12, atol=1e-12)


def test_split_merge_identity():
    """Split-K partials (m, l, acc) merged by log-sum-exp equal attention over all keys -- the kernels' merge."""
    rng = np.random.default_rng(5)
    n, d = 300, 16
    q = rng.standard_normal(d)
    k = rng.standard_normal((n, d))
    v = rng.standard_normal((n, d))
    s = k @ q * 0.25
    full = (np.exp(s - s.max()) @ v) / np.exp(s - s.max()).sum()
    parts = []
    for lo, hi in ((0, 64), (64, 64), (64, 250), (250, 300)):  # one split empty
        if hi == lo:
            parts.append((-np.inf, 0.0, np.zeros(d)))
            continue
        m = s[lo:hi].max()
        p = np.exp(s[lo:hi] - m)
        parts.append((m, p.sum(), p @ v[lo:hi]))
    top = max(m for m, _, _ in parts)
    w = [0.0 if m == -np.inf else math.exp(m - top) for m, _, _ in parts]
    merged = sum(wi * a for wi, (_, _, a) in zip(w, parts)) / sum(wi * l for wi, (_, l, _) in zip(w, parts))
    np.testing.assert_allclose(merged, full, rtol=1e-12, atol=1e-12)


def test_one_query_is_decode_attention():
    rng = np.random.default_rng(6)
    q = rng.standard_normal((3, 2, 8))
    kc = rng.standard_normal((3, 2, 20, 8))
    vc = rng.standard_normal((3, 2, 20, 8))
    lengths = np.array([20, 1, 0])
    out = ov.verify_attention(q, kc, vc, lengths, 1, 0.5)
    for r, n in enumerate(lengths):
        if n == 0:
            assert np.all(out[r] == 0)
            continue
        ref = torch.softmax(torch.from_numpy(q[r])[:, None] @ torch.from_numpy(kc[r, :, :n]).transpose(-1, -2) * 0.5, -1)
        np.testing.assert_allclose(out[r], (ref @ torch.from_numpy(vc[r, :, :n]))[:, 0].numpy(), rtol=1e-12)


def _beam_case(seed, groups=3, beams=2, heads=2, d=8, cap=20, gcap=9):
    rng = np.random.default_rng(seed)
    rows = groups * beams
    q = rng.standard_normal((rows, heads, d))
    kc, vc = rng.standard_normal((2, groups + 1, heads, cap, d))
    kg, vg = rng.standard_normal((2, rows + 2, heads, gcap, d))
    ptr = rng.integers(0, rows + 2, (rows, gcap)).astype(np.int32)
    return q, kc, vc, kg, vg, ptr


def test_beam_attention_reductions():
    """One beam without generated keys is decode attention; context-free rows whose pointers name themselves are
    decode attention over their own generated rows."""
    q, kc, vc, kg, vg, ptr = _beam_case(7, beams=1)
    ctx_len = np.array([20, 4, 0])
    out = ov.beam_attention(q, kc, vc, ctx_len, kg, vg, ptr, np.zeros(3, np.int64), 1, 0.3)
    np.testing.assert_allclose(out, ov.verify_attention(q, kc, vc, ctx_len, 1, 0.3), rtol=1e-12, atol=1e-15)
    q, kc, vc, kg, vg, ptr = _beam_case(8, beams=3)
    rows = q.shape[0]
    own = np.repeat(np.arange(rows, dtype=np.int32)[:, None], ptr.shape[1], 1)
    gen_len = np.array([9, 1, 0, 5, 3, 7, 2, 8, 4])
    out = ov.beam_attention(q, kc, vc, np.zeros(3, np.int64), kg, vg, own, gen_len, 3, 0.3)
    want = ov.verify_attention(q, kg[:rows], vg[:rows], gen_len, 1, 0.3)
    np.testing.assert_allclose(out, want, rtol=1e-12, atol=1e-15)


def test_beam_attention_is_gather_then_masked_softmax():
    """The unfused formulation: every row gathers its full context and generated caches, masks what it may not see
    and takes one softmax (src/omniasr_trt/beam.py:113-125), in torch float64."""
    q, kc, vc, kg, vg, ptr = _beam_case(9, groups=4, beams=3)
    ctx_len = np.array([20, 13, 1, 0])
    gen_len = np.array([9, 0, 4, 6, 2, 1, 0, 9, 3, 0, 0, 0])
    out = ov.beam_attention(q, kc, vc, ctx_len, kg, vg, ptr, gen_len, 3, 0.3)
    t = {k: torch.from_numpy(v) for k, v in dict(q=q, kc=kc, vc=vc, kg=kg, vg=vg).items()}
    rows, cap, gcap = q.shape[0], kc.shape[2], kg.shape[2]
    group = torch.arange(rows) // 3
    src = torch.from_numpy(ptr).long()
    j = torch.arange(gcap)
    k = torch.cat([t["kc"][group], t["kg"][src, :, j].transpose(1, 2)], 2)  # [R, H, C + G, D]
    v = torch.cat([t["vc"][group], t["vg"][src, :, j].transpose(1, 2)], 2)
    allowed = torch.cat([torch.arange(cap)[None] < torch.from_numpy(ctx_len)[group, None],
                         j[None] < torch.from_numpy(gen_len)[:, None]], 1)
    sc = (t["q"][:, :, None, :] @ k.transpose(-1, -2)) * 0.3
    w = torch.softmax(sc.masked_fill(~allowed[:, None, None], float("-inf")), -1).nan_to_num(0.0)
    np.testing.assert_allclose(out, (w @ v)[:, :, 0].numpy(), rtol=1e-12, atol=1e-14)
    assert np.all(out[9:] == 0)  # the finished group reads nothing


# ---------------------------------------------------------------------------------------------- argmax

def test_argmax_oracle_matches_torch_log_softmax():
    """The oracle's float32 log-probabilities against PyTorch's float32 ``F.log_softmax`` (CPU) to a few ulps, and its
    bf16 argmax against the argmax of PyTorch's values rounded to bf16 -- equal on every row whose result does not
    hinge on the last bits of the log-sum-exp."""
    g = torch.Generator().manual_seed(7)
    x = torch.randn(2000, 10288, generator=g).to(torch.bfloat16)
    xn = _bf16_np(x)
    ref = F.log_softmax(x.float(), -1).numpy()
    y = ov.log_softmax_f32(xn)
    assert np.abs(y - ref).max() <= 4 * np.spacing(np.float32(16.0))
    want = bf16.round_bf16(ref).argmax(-1)
    got = ov.log_softmax_argmax(xn, "bf16")
    fragile = ov.argmax_is_fragile(xn, "bf16")
    assert not ((got != want) & ~fragile).any()
    assert fragile.mean() < 0.01
    # the bucket rule matters: the plain argmax of the logits disagrees on about 1% of rows
    assert 0.003 < (xn.argmax(-1) != got).mean() < 0.03


def test_torch_cpu_bf16_log_softmax_is_another_rounding():
    """PyTorch's CPU kernel for bf16 input keeps the sum and its log in bf16 (its buffers have the input's type):
    y = bf16((x - m) - bf16(log(bf16(sum)))).  The reference runs the GPU kernel, which keeps them in fp32."""
    g = torch.Generator().manual_seed(8)
    x = torch.randn(200, 10288, generator=g).to(torch.bfloat16)
    xn = _bf16_np(x)
    m = xn.max(-1, keepdims=True)
    s = np.exp(xn - m).astype(np.float32).sum(-1, keepdims=True, dtype=np.float64).astype(np.float32)
    cpu_rule = bf16.round_bf16((xn - m) - bf16.round_bf16(np.log(bf16.round_bf16(s))))
    np.testing.assert_array_equal(F.log_softmax(x, -1).float().numpy(), cpu_rule)


def test_argmax_fp32_and_planted():
    g = torch.Generator().manual_seed(8)
    x = torch.randn(500, 37, generator=g)
    np.testing.assert_array_equal(ov.log_softmax_argmax(x.numpy(), "f32"), F.log_softmax(x, -1).argmax(-1).numpy())
    # config 1: a planted argmax 1.0 above the row maximum is the argmax whatever the rounding
    y = torch.randn(5, 10288, generator=g).to(torch.bfloat16)
    drafts = [11, 222, 3333, 4444]
    for r in range(2):
        y[r, drafts[r]] = y[r].float().max() + 1.0
    got = ov.log_softmax_argmax(_bf16_np(y), "bf16")
    assert got[0] == 11 and got[1] == 222


# ---------------------------------------------------------------------------------------------- accept

def test_accept_golden_vectors():
    """The reference's own ``_accept`` (run under Triton's interpreter) on 24 random states."""
    z = np.load(GOLD / "accept_golden.npz")
    for c in range(int(z["cases"])):
        p = f"c{c}_"
        out, tok, last = z[p + "out"].copy(), z[p + "tok"].copy(), z[p + "last"].copy()
        done, dn = z[p + "done"].copy(), z[p + "draft_next"].copy()
        ov.accept(z[p + "tokens"], z[p + "nxt"], out, tok, last, done, dn, z[p + "start"], z[p + "use_draft"],
                  int(z[p + "limit"]), int(z[p + "eos"]))
        for name, got in (("out", out), ("tok", tok), ("last", last), ("done", done), ("draft_next", dn)):
            np.testing.assert_array_equal(got, z[p + name + "_after"], err_msg=f"case {c} {name}")


def test_accept_known_answers():
    """Planted: the first two drafts match -> n = 2, three tokens kept, last += 3; EOS and the limit cut a step."""
    t0, d = 9, [5, 6, 7, 8]
    tokens = np.array([[t0] + d] * 3)
    nxt = np.array([[5, 6, 4, 8, 3], [5, 2, 7, 8, 3], [5, 6, 7, 8, 3]])
    out = np.full((3, 64), 1, np.int32)
    tok, last = np.array([t0] * 3), np.array([10, 20, 30])
    done = np.zeros(3, bool)
    dn, start, use = np.array([100, 100, 100]), np.array([50, 50, 50]), np.array([True, False, True])
    ov.accept(tokens, nxt, out, tok, last, done, dn, start, use, limit=33, eos=2)
    assert list(out[0, 11:14]) == [5, 6, 4] and last[0] == 13 and tok[0] == 4 and not done[0] and dn[0] == 53
    assert list(out[1, 21:23]) == [5, 2] and last[1] == 22 and tok[1] == 2 and done[1] and dn[1] == 102
    # row 2: everything matches, but position 31 + 2 = 33 >= limit stops at j = 2
    assert list(out[2, 31:34]) == [5, 6, 7] and last[2] == 33 and done[2] and dn[2] == 53


def test_accept_one_token_is_the_greedy_update():
    rng = np.random.default_rng(9)
    for _ in range(50):
        b = 12
        nxt = rng.integers(0, 6, b)
        last = rng.integers(0, 60, b)
        done = rng.random(b) < 0.3
        out = rng.integers(3, 9, (b, 64)).astype(np.int32)
        tok = rng.integers(3, 9, b)
        a = [x.copy() for x in (out, tok, last, done)]
        ov.accept(tok[:, None], nxt[:, None], a[0], a[1], a[2], a[3], None, None, None, limit=40, eos=2)
        g = [x.copy() for x in (out, tok, last, done)]
        ov.greedy_update(nxt, g[0], g[1], g[2], g[3], limit=40, eos=2)
        for x, y in zip(a, g):
            np.testing.assert_array_equal(x, y)


# ---------------------------------------------------------------------------------------------- propose

def test_propose_golden_vectors():
    """The reference's ``_propose`` kernel and ``reference_propose`` (which agreed) on 12 trials."""
    z = np.load(GOLD / "propose_golden.npz")
    const = z["constants"]
    assert list(const[:5]) == [NGRAM, BEHIND, AHEAD, SELF_WINDOW, SELF_MIN]
    assert [tuple(const[5 + 2 * i: 7 + 2 * i]) for i in range(4)] == list(REACH)
    for t in range(int(z["trials"])):
        p = f"t{t}_"
        prop, use, start = ov.propose(z[p + "out"], z[p + "draft"], z[p + "draft_len"], z[p + "last"], z[p + "first"],
                                      z[p + "next"], int(z[p + "k"]), NGRAM, BEHIND, AHEAD, REACH, W, SW, SELF_MIN)
        np.testing.assert_array_equal(prop, z[p + "prop"], err_msg=f"trial {t}")
        np.testing.assert_array_equal(use, z[p + "use_draft"], err_msg=f"trial {t}")
        np.testing.assert_array_equal(start, z[p + "start"], err_msg=f"trial {t}")


def _tiny_propose_case(rng, b=6, cap=80, dcap=60, vocab=4):
    out = rng.integers(3, 3 + vocab, (b, cap)).astype(np.int32)
    first = rng.integers(0, 20, b)
    last = np.minimum(first + rng.integers(0, 50, b), cap - 1)
    out[np.arange(cap)[None, :] < first[:, None]] = 1
    dlen = rng.integers(0, dcap + 1, b)
    draft = rng.integers(3, 3 + vocab, (b, dcap)).astype(np.int32)
    draft[np.arange(dcap)[None, :] >= dlen[:, None]] = -1
    nxt = (rng.random(b) * (dlen + 6)).astype(np.int64)
    return out, draft, dlen, last, first, nxt


def test_propose_brute_force():
    rng = np.random.default_rng(10)
    for trial in range(60):
        case = _tiny_propose_case(rng, vocab=2 + trial % 4)
        k, ngram = 1 + trial % 5, 2 + trial % 6
        behind, ahead = 3 + trial % 7, 5 + trial % 9
        width = 1 << (behind + ahead).bit_length()
        reach = ((0, 1), (2, 2), (4, 3), (6, 4))
        a = ov.propose(*case, k, ngram, behind, ahead, reach, width, 16, 2)
        b = ov.propose_loops(*case, k, ngram, behind, ahead, reach, width, 16, 2)
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y, err_msg=f"trial {trial}")


def test_propose_invariants():
    # a perfect draft: the generated tokens are the draft's first tokens -> propose the next ones from the draft
    draft_tokens = list(range(10, 60))
    out = np.full((1, 128), 1, np.int32)
    first, last = 20, 29  # 10 generated tokens = draft[0..9]
    out[0, first:last + 1] = draft_tokens[:10]
    draft = np.full((1, 64), -1, np.int32)
    draft[0, :50] = draft_tokens
    prop, use, start = ov.propose(out, draft, np.array([50]), np.array([last]), np.array([first]), np.array([10]),
                                  4, NGRAM, BEHIND, AHEAD, REACH, W, SW, SELF_MIN)
    assert use[0] and list(prop[0]) == draft_tokens[10:14] and start[0] == 10
    # a repetition loop and no draft: continue with the period
    out = np.full((1, 128), 1, np.int32)
    loop = [7, 8, 9] * 10
    out[0, 0:30] = loop
    prop, use, _ = ov.propose(out, np.full((1, 8), -1, np.int32), np.array([0]), np.array([29]), np.array([0]),
                              np.array([0]), 5, NGRAM, BEHIND, AHEAD, REACH, W, SW, SELF_MIN)
    assert not use[0] and list(prop[0]) == [7, 8, 9, 7, 8]


def test_spec_prepare_rules():
    rng = np.random.default_rng(11)
    out, draft, dlen, last, first, nxt = _tiny_propose_case(rng, b=5)
    tok = rng.integers(3, 7, 5)
    done = np.array([False, True, False, True, False])
    tokens, pos, slots, lengths, use, start = ov.spec_prepare(out, draft, dlen, last, first, nxt, tok, done, 60, 3,
                                                              NGRAM, 4, 6, REACH, 16, 16, 2)
    prop, use2, start2 = ov.propose(out, draft, dlen, last, first, nxt, 3, NGRAM, 4, 6, REACH, 16, 16, 2)
    np.testing.assert_array_equal(tokens[:, 0], tok)
    np.testing.assert_array_equal(tokens[:, 1:], prop)
    for b in range(5):
        want = [min(last[b], 59)] * 4 if done[b] else [min(last[b] + 1 + j, 59) for j in range(4)]
        assert list(pos[b * 4:(b + 1) * 4]) == want
        assert lengths[b] == (0 if done[b] else last[b] + 2)
    np.testing.assert_array_equal(slots, np.repeat(np.arange(5), 4))


# ---------------------------------------------------------------------------------------------- drafts, host rules

def test_frames_to_draft_matches_loop():
    from omniasr_trt_amd import llm

    rng = np.random.default_rng(12)
    for trial in range(40):
        frames = rng.integers(0, 6, rng.integers(0, 400))
        seg_samples = 2000 + 320 * int(rng.integers(0, 5))
        for seg in range(3):
            assert llm.frames_to_draft(frames, seg, seg_samples) == ov.frames_to_draft(frames, seg, seg_samples)
    # hand-computed: segment 1 of 6400-sample segments is frames [20, 40), window [0, 90) -> 25 frames before
    frames = np.array([0] * 5 + [3, 3, 4, 0, 4] + [5] * 15 + [6, 2, 6] + [7] * 10)
    ids, before = llm.frames_to_draft(frames, 1, 6400)
    assert ids == [3, 4, 4, 5, 6, 6, 7] and before == 4


def test_early_stop_rule_known_answers():
    from omniasr_trt_amd import llm

    out = np.full(1000, 1, dtype=np.int32)
    out[300:] = 7
    assert llm.compression_ratio(out[400:500]) > 4.0
    assert llm.compression_ratio(out[400:500]) == oref.compression_ratio(out[400:500])
    assert llm.early_stop_index(out, 240, 600, ctx=300) == 500
    assert llm.early_stop_index(out, 240, 499, ctx=300) is None
    assert llm.early_stop_index(out, 240, 800, ctx=420) == 750


# ---------------------------------------------------------------------------------------------- beam search

def _small_decoder(seed, vocab=12, peak=4.0):
    from omniasr_trt_amd.modeling import DecoderConfig, DecoderModel

    torch.manual_seed(seed)
    cfg = DecoderConfig(model_dim=32, num_layers=2, num_heads=2, ffn_dim=24, vocab_size=vocab, num_langs=5,
                        max_seq_len=512)
    m = DecoderModel(cfg).double().eval()
    with torch.no_grad():
        for p in m.parameters():
            p.normal_(0, 0.5)
        m.final_proj.weight.mul_(peak)
    return oref.Fp64Decoder(m)


def _contexts(seed, lengths):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(n, 32, generator=g, dtype=torch.float64) for n in lengths]


def test_one_beam_is_greedy():
    dec = _small_decoder(11)
    for c in _contexts(1, (5, 30, 17)):
        greedy = oref.greedy_reference(dec, c)
        assert oref.beam_reference(dec, c, 1) == greedy
        assert oref.beam_reference(dec, c, 1, length_norm=True) == greedy  # a monotone map of one row's offers


def test_beam_search_two_tokens_brute_force():
    """As many beams as tokens, stopped after two tokens: every first token survives the first step, so the result is
    the best of all two-token sequences (a sequence that starts with EOS keeps EOS's score)."""
    dec = _small_decoder(13, peak=1.0)  # flatter distributions: greedy misses the best pair in 4 of these 10
    vocab = dec.sd["final_proj.weight"].size(0)
    differs = 0
    for c in _contexts(2, (6, 11, 3, 25, 9, 14, 7, 8, 19, 4)):
        n = c.size(0)
        cache = [None] * dec.layers
        dec.forward(c[: n - 1], torch.arange(n - 1), cache)
        lp1 = F.log_softmax(dec.logits(dec.forward(c[n - 1][None], torch.tensor([n - 1]), cache)[0]), -1)
        best, best_seq = -math.inf, None
        for a in range(vocab):
            if a == oref.EOS:
                score, seq = float(lp1[a]), (a, oref.EOS)
            else:
                branch = [(k.clone(), v.clone()) for k, v in cache]
                lp2 = F.log_softmax(dec.logits(dec.forward(dec.embed(a)[None], torch.tensor([n]), branch)[0]), -1)
                b = int(lp2.argmax())
                score, seq = float(lp1[a] + lp2[b]), (a, b)
            if score > best:
                best, best_seq = score, seq
        want = [t for t in best_seq if t not in (oref.PAD, oref.BOS, oref.EOS)]
        assert oref.beam_reference(dec, c, vocab, limit=n) == want
        differs += oref.greedy_reference(dec, c, limit=n) != want
    assert differs >= 2  # the search found sequences greedy decoding misses


# ---------------------------------------------------------------------------------------------- beam step bookkeeping

def _beam_state(rng, groups, beams, vocab, cols, score_dtype=np.float32):
    rows = groups * beams
    st = dict(
        ctx=rng.integers(1, 500, groups).astype(np.int64),
        k_step=rng.integers(1, cols, groups).astype(np.int64),
        group_done=rng.random(groups) < 0.3,
        ptr=rng.integers(0, rows, (rows, cols)).astype(np.int32),
        hist=rng.integers(0, vocab, (rows, cols + 1)).astype(np.int32),
        ended=rng.random(rows) < 0.3,
        score=(rng.standard_normal(rows) * 3).astype(score_dtype),
        count=rng.integers(0, 50, rows).astype(np.int64),
        tok=rng.integers(0, vocab, rows).astype(np.int64),
    )
    best = np.sort(rng.standard_normal((groups, beams)).astype(score_dtype), axis=1)[:, ::-1].copy()
    flat = rng.integers(0, beams * vocab, (groups, beams)).astype(np.int64)
    flat[:, 0] = flat[:, 0] - flat[:, 0] % vocab + 2  # every group's best: EOS (2)
    if beams > 1:
        flat[:, 1] = flat[:, 1] - flat[:, 1] % vocab + 1  # the second: PAD (1)
    return st, best, flat


def _beam_take_over_torch(best, flat, vocab, st, limit, eos, pad):
    """The reference's vectorised formulation of the step after the top-k (src/omniasr_trt/beam.py:170-187), on
    CPU tensors: the check the row-by-row oracle is held to."""
    s, n = best.shape
    r = s * n
    t = {k: torch.from_numpy(v.copy()) for k, v in st.items()}
    best, flat = torch.from_numpy(best.copy()), torch.from_numpy(flat.copy())
    rows = torch.arange(r)
    group = rows // n
    live = ~t["group_done"][group]
    k = t["k_step"][group]
    parent = torch.where(live, (flat // vocab + torch.arange(s)[:, None] * n).view(-1), rows)
    new = torch.where(live, (flat % vocab).view(-1), t["tok"])
    ptr, hist = t["ptr"], t["hist"]
    ptr.copy_(ptr[parent])
    hist.copy_(hist[parent])
    p_ended, p_score, p_count = t["ended"][parent], t["score"][parent], t["count"][parent]
    new = torch.where(p_ended, eos, new)
    hist.scatter_(1, k[:, None], torch.where(live, new, hist.gather(1, k[:, None])[:, 0].long())[:, None]
                  .to(hist.dtype))
    t["score"].copy_(torch.where(live & ~p_ended, best.view(-1), p_score))
    t["count"].copy_(p_count + (live & ~p_ended & (new != pad) & (new != eos)).long())
    t["ended"].copy_(torch.where(live, new == eos, p_ended))
    t["tok"].copy_(new)
    all_ended = t["ended"].view(s, n).all(-1)
    t["k_step"].copy_(t["k_step"] + (~t["group_done"]).long())
    t["group_done"] |= all_ended | (t["ctx"] - 1 + t["k_step"] - 1 >= limit)
    return {k: v.numpy() for k, v in t.items()}


def test_beam_take_over_oracle_vs_the_vectorised_step():
    rng = np.random.default_rng(31)
    for trial in range(60):
        groups, beams, vocab, cols = int(rng.integers(1, 9)), int(rng.integers(1, 17)), int(rng.integers(3, 40)), 24
        dt = np.float64 if trial % 3 == 0 else np.float32
        st, best, flat = _beam_state(rng, groups, beams, vocab, cols, dt)
        limit = int(rng.integers(5, 600))
        want = _beam_take_over_torch(best, flat, vocab, st, limit, 2, 1)
        got = {k: v.copy() for k, v in st.items()}
        ov.beam_take_over(best, flat, vocab, got["ptr"], got["hist"], got["ended"], got["score"], got["count"],
                          got["tok"], got["k_step"], got["group_done"], got["ctx"], limit, 2, 1)
        for key in want:
            np.testing.assert_array_equal(got[key], want[key], err_msg=f"trial {trial}: {key}")


def test_beam_take_over_known_answer():
    """Two groups of three beams, vocabulary 10: group 0 live (its row 1 had ended), group 1 finished."""
    best = np.array([[-1.0, -2.0, -3.0], [-0.5, -0.6, -0.7]], np.float32)
    flat = np.array([[1 * 10 + 7, 0 * 10 + 2, 2 * 10 + 5], [0, 11, 22]], np.int64)  # (parent, token)
    ptr = np.arange(6 * 4, dtype=np.int32).reshape(6, 4)
    hist = np.arange(100, 100 + 6 * 5, dtype=np.int32).reshape(6, 5)
    ended = np.array([False, True, False, True, False, False])
    score = np.array([-0.1, -0.2, -0.3, -0.4, -0.5, -0.6], np.float32)
    count = np.array([3, 4, 5, 6, 7, 8], np.int64)
    tok = np.array([9, 9, 9, 4, 5, 6], np.int64)
    k_step = np.array([2, 3], np.int64)
    group_done = np.array([False, True])
    ctx = np.array([10, 10], np.int64)
    ov.beam_take_over(best, flat, 10, ptr, hist, ended, score, count, tok, k_step, group_done, ctx, 8188, 2, 1)
    # row 0: parent 1 (ended) -> EOS, score and count of the parent, still ended
    # row 1: parent 0 token 2 = EOS -> ended, count unchanged, score -2.0
    # row 2: parent 2 token 5 -> score -3.0, count 6
    np.testing.assert_array_equal(tok[:3], [2, 2, 5])
    np.testing.assert_array_equal(ended[:3], [True, True, False])
    np.testing.assert_array_equal(score[:3], np.array([-0.2, -2.0, -3.0], np.float32))
    np.testing.assert_array_equal(count[:3], [4, 3, 6])
    np.testing.assert_array_equal(ptr[:3], np.arange(24, dtype=np.int32).reshape(6, 4)[[1, 0, 2]])
    want_hist = np.arange(100, 130, dtype=np.int32).reshape(6, 5)[[1, 0, 2]].copy()
    want_hist[:, 2] = [2, 2, 5]
    np.testing.assert_array_equal(hist[:3], want_hist)
    assert k_step[0] == 3 and not group_done[0]
    # group 1 is finished: its rows keep their state; tok becomes EOS where the row had ended
    np.testing.assert_array_equal(tok[3:], [2, 5, 6])
    np.testing.assert_array_equal(ptr[3:], np.arange(24, dtype=np.int32).reshape(6, 4)[3:])
    np.testing.assert_array_equal(score[3:], np.array([-0.4, -0.5, -0.6], np.float32))
    assert k_step[1] == 3 and group_done[1]


def test_beam_prepare_oracle():
    rng = np.random.default_rng(32)
    for trial in range(30):
        groups, beams, cols = int(rng.integers(1, 9)), int(rng.integers(1, 17)), 20
        ctx = rng.integers(1, 500, groups).astype(np.int64)
        k_step = rng.integers(0, cols + 3, groups).astype(np.int64)
        done = rng.random(groups) < 0.3
        ptr = rng.integers(0, 99, (groups * beams, cols)).astype(np.int32)
        want_ptr = ptr.copy()
        got = ov.beam_prepare(groups, beams, ctx, k_step, done, ptr)
        # the reference's vectorised formulation (src/omniasr_trt/beam.py:133-145)
        r = groups * beams
        group = np.arange(r) // beams
        live = ~done[group]
        k = k_step[group]
        j = np.maximum(k - 1, 0)
        np.testing.assert_array_equal(got[0], ctx[group] - 1 + k)
        np.testing.assert_array_equal(got[1], j)
        np.testing.assert_array_equal(got[2], np.where(done, 0, ctx))
        np.testing.assert_array_equal(got[3], np.where(live, k, 0))
        for row in range(r):
            if live[row] and j[row] < cols:
                want_ptr[row, j[row]] = row
        np.testing.assert_array_equal(ptr, want_ptr)

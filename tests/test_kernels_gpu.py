"""The HIP kernels against the oracle on an MI355X, through the C ABI (the ``kernels`` shim): bit-exact for RoPE +
append, argmax indices, acceptance and proposal; 2e-2 abs / 1e-2 rel (bf16) or 1e-4 (fp32) for attention."""

import sys
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import bf16 as obf
from oracle import verify as ov
from omniasr_trt_amd import kernels, modeling

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).parent / "golden"
NGRAM, BEHIND, AHEAD, SELF_WINDOW, SELF_MIN = 8, 64, 160, 256, 3
REACH = ((1, 1), (4, 2), (12, 4), (40, 6))


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def npf(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def gen(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------------------------------------- RoPE + append

def _rope_case(cuda, dtype, d, h, n, rows, s, pos, slots=None, cache_pos=None, seed=0):
    g = gen(seed)
    qkv = torch.randn(n, 3 * h * d, generator=g).to(dtype)
    cfg = modeling.DecoderConfig(model_dim=h * d, num_heads=h)
    cs = modeling.rope_table(cfg)  # one table, the same bits on both sides
    kc = torch.randn(rows, h, s, d, generator=g).to(dtype)
    vc = torch.randn(rows, h, s, d, generator=g).to(dtype)
    kd, vd = kc.to(cuda), vc.to(cuda)
    say(f"rope_kv dtype={dtype} d={d} h={h} n={n} rows={rows} s={s}")
    q = kernels.rope_kv(qkv.to(cuda), cs.to(cuda), pos.to(cuda), kd, vd, h,
                        None if slots is None else slots.to(cuda), None if cache_pos is None else cache_pos.to(cuda))
    torch.cuda.synchronize()
    okc, ovc = npf(kc), npf(vc)
    tag = "bf16" if dtype == torch.bfloat16 else "f32"
    want_q = ov.rope_kv(npf(qkv), cs.numpy(), pos.numpy(), okc, ovc, h,
                        None if slots is None else slots.numpy(), None if cache_pos is None else cache_pos.numpy(), tag)
    np.testing.assert_array_equal(npf(q), want_q)
    r = np.arange(n) if slots is None else slots.numpy()
    c = pos.numpy() if cache_pos is None else cache_pos.numpy()
    # the written positions (unique ones: the oracle's last writer equals the kernel's only writer)
    np.testing.assert_array_equal(npf(kd[torch.as_tensor(r), :, torch.as_tensor(c)]), okc[r, :, c])
    np.testing.assert_array_equal(npf(vd[torch.as_tensor(r), :, torch.as_tensor(c)]), ovc[r, :, c])
    # everything else untouched
    mask = torch.zeros(rows, h, s, dtype=torch.bool)
    mask[torch.as_tensor(r), :, torch.as_tensor(c)] = True
    assert torch.equal(kd.cpu()[~mask], kc[~mask]) and torch.equal(vd.cpu()[~mask], vc[~mask])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rope_kv_config2(cuda, dtype):
    """Config 2: 8 slots x 5 new tokens, 32 heads x 128, cache 4096, positions = current lengths U[200, 2000]."""
    g = gen(1002)
    lengths = torch.randint(200, 2001, (8,), generator=g)
    pos = (lengths[:, None] + torch.arange(5)).reshape(-1)
    slots = torch.arange(8).repeat_interleave(5)
    _rope_case(cuda, dtype, 128, 32, 40, 8, 4096, pos, slots, seed=1002)


@pytest.mark.parametrize("dtype,d,h", [(torch.bfloat16, 512, 8), (torch.float32, 512, 8), (torch.float32, 16, 2),
                                       (torch.bfloat16, 64, 4)])
def test_rope_kv_head_dims(cuda, dtype, d, h):
    pos = torch.tensor([0, 7, 299, 150, 31])
    _rope_case(cuda, dtype, d, h, 5, 7, 300, pos, seed=3)
    # scattered cache rows (prefill of refilled slots) and explicit cache positions (beam search)
    _rope_case(cuda, dtype, d, h, 5, 7, 300, pos, slots=torch.tensor([6, 0, 3, 5, 1]), seed=4)
    _rope_case(cuda, dtype, d, h, 5, 7, 300, pos, slots=torch.tensor([6, 0, 3, 5, 1]),
               cache_pos=torch.tensor([1, 2, 3, 4, 5]), seed=5)


def test_rope_kv_prefill_size(cuda):
    """The prefill shape of config 2: 8 contexts x 2048 tokens through one launch."""
    n = 8 * 2048
    pos = torch.arange(2048).repeat(8)
    slots = torch.arange(8).repeat_interleave(2048)
    _rope_case(cuda, torch.bfloat16, 128, 32, n, 8, 2048, pos, slots, seed=6)


# ---------------------------------------------------------------------------------------------- verify attention

def _attn_case(cuda, dtype, b, h, d, t, cap, lengths, keys, seed, tol, **launch):
    g = gen(seed)
    kc = torch.randn(b + 1, h, cap, d, generator=g).to(dtype)
    vc = torch.randn(b + 1, h, cap, d, generator=g).to(dtype)
    q = torch.randn(b * t, h, d, generator=g).to(dtype)
    say(f"verify attention dtype={dtype} b={b} h={h} d={d} t={t} keys={keys} lengths={lengths.tolist()[:8]} {launch}")
    out = kernels.draft_attention(q.to(cuda), kc.to(cuda), vc.to(cuda), lengths.to(cuda), t, keys, d ** -0.5,
                                  **launch)
    torch.cuda.synchronize()
    want = ov.verify_attention(npf(q), npf(kc), npf(vc), lengths.numpy(), t, d ** -0.5)
    np.testing.assert_allclose(npf(out), want, atol=tol[0], rtol=tol[1])
    return out


BF16_TOL = (2e-2, 1e-2)  # the north star's bound for bf16 storage with fp32 accumulation
F32_TOL = (1e-4, 1e-4)


@pytest.mark.parametrize("t", [1, 3, 5, 9, 16])
def test_verify_attention_bf16(cuda, t):
    lengths = torch.tensor([600, 257, 1, 0])  # 0: a finished row (query i then sees keys [0, i))
    _attn_case(cuda, torch.bfloat16, 4, 8, 128, t, 700, lengths, 640, 2, BF16_TOL)
    _attn_case(cuda, torch.bfloat16, 4, 8, 512, t, 700, lengths, 640, 3, BF16_TOL)
    _attn_case(cuda, torch.bfloat16, 4, 4, 256, t, 700, lengths, 640, 5, BF16_TOL)  # two 128-dimension slices


@pytest.mark.parametrize("b,keys", [(1, 256), (3, 1024), (8, 2048), (16, 512)])
def test_decode_attention_reference_cases(cuda, b, keys):
    """The reference's own decode-attention cases (src tests/test_kernels.py:42-55): fp32, 8 heads x 512, a cache of
    2048 positions, lengths U[1, keys] with row 0 at ``keys`` (the whole bucket; at 2048 the whole cache), within the
    reference's tolerance of 2e-5 of the fp64 oracle."""
    g = gen(b * 7 + keys)
    h, d, cap = 8, 512, 2048
    kc = torch.randn(b + 1, h, cap, d, generator=g)
    vc = torch.randn(b + 1, h, cap, d, generator=g)
    q = torch.randn(b, h, d, generator=g)
    lengths = torch.randint(1, keys + 1, (b,), generator=g)
    lengths[0] = keys
    say(f"decode_attention reference case b={b} keys={keys}")
    out = kernels.decode_attention(q.to(cuda), kc.to(cuda), vc.to(cuda), lengths.to(cuda), keys, d ** -0.5)
    torch.cuda.synchronize()
    want = ov.verify_attention(npf(q), npf(kc)[:b], npf(vc)[:b], lengths.numpy(), 1, d ** -0.5)
    np.testing.assert_allclose(npf(out), want, atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("dtype,rows,heads,d", [(torch.bfloat16, 8, 32, 128), (torch.bfloat16, 3, 4, 128),
                                                 (torch.bfloat16, 8, 8, 512), (torch.float32, 5, 4, 64),
                                                 (torch.float32, 4, 2, 512)])
def test_decode_attention_shim(cuda, dtype, rows, heads, d):
    """``kernels.decode_attention`` through its own signature, as the reference's one-token step calls it
    (src/omniasr_trt/decode.py:203-204: ``decode_attention(q, self.k[i], self.v[i], lengths, keys, scale)`` on a
    layer's [max_batch, H, S, D] cache, q [B, H, D]), and with the reference's Triton settings passed explicitly
    (accepted and ignored) and a ``chunk`` override: against the oracle's attention at one query per row, a row of
    length 0 giving zeros (src/omniasr_trt/kernels.py:210)."""
    g = gen(rows * 100 + heads + d)
    cap, max_batch = 1536, rows + 3
    layers_k = torch.randn(2, max_batch, heads, cap, d, generator=g).to(dtype)
    layers_v = torch.randn(2, max_batch, heads, cap, d, generator=g).to(dtype)
    lengths = torch.randint(1, 1400, (rows,), generator=g)
    lengths[rows // 2] = 0
    lengths[0] = 1
    keys = -(-int(lengths.max()) // 256) * 256
    q = torch.randn(rows, heads, d, generator=g).to(dtype)
    kd, vd, qd, ld = layers_k.to(cuda), layers_v.to(cuda), q.to(cuda), lengths.to(cuda)
    want = ov.verify_attention(npf(q), npf(layers_k[1]), npf(layers_v[1]), lengths.numpy(), 1, d ** -0.5)
    tol = BF16_TOL if dtype == torch.bfloat16 else F32_TOL
    outs = []
    for kw in ({}, {"block": 64, "warps": 8, "stages": 2, "programs": 264}, {"chunk": 256}):
        say(f"decode_attention dtype={dtype} rows={rows} heads={heads} d={d} keys={keys} {kw}")
        out = kernels.decode_attention(qd, kd[1], vd[1], ld, keys, d ** -0.5, **kw)
        torch.cuda.synchronize()
        assert out.shape == q.shape and out.dtype == dtype
        np.testing.assert_allclose(npf(out), want, atol=tol[0], rtol=tol[1])
        assert not npf(out[rows // 2]).any()  # the empty row: zeros
        outs.append(out)
    assert torch.equal(outs[0], outs[1])  # the Triton settings change nothing
    assert int(kernels._counters[torch.cuda.current_device()].abs().sum()) == 0


@pytest.mark.parametrize("t,d", [(20, 512), (32, 512), (32, 256)])
def test_verify_attention_wide_heads_up_to_32_queries(cuda, t, d):
    """Head dims 256 / 512 take up to 32 queries per row (two 16-query groups per wave): against the oracle, both
    merge modes; a 128-wide head with more than 16 queries is refused."""
    lengths = torch.tensor([600, 257, 1, 0])
    a = _attn_case(cuda, torch.bfloat16, 4, 2, d, t, 700, lengths, 640, 11, BF16_TOL, separate=True)
    b = _attn_case(cuda, torch.bfloat16, 4, 2, d, t, 700, lengths, 640, 11, BF16_TOL, separate=False)
    torch.testing.assert_close(a.float(), b.float(), atol=1e-2, rtol=1e-2)
    q = torch.zeros(2 * 17, 2, 128, dtype=torch.bfloat16, device=cuda)
    kc = torch.zeros(2, 2, 256, 128, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(RuntimeError):
        kernels.draft_attention(q, kc, kc, torch.tensor([5, 9], device=cuda), 17, 256, 0.1)


@pytest.mark.parametrize("width,d,b,h", [(1, 128, 3, 4), (15, 128, 3, 4), (64, 128, 3, 4), (97, 128, 3, 4),
                                         (300, 128, 3, 4), (1, 512, 3, 4), (15, 512, 3, 4), (96, 512, 3, 4),
                                         (97, 512, 3, 4), (300, 512, 3, 4), (1, 256, 3, 4), (192, 256, 3, 4),
                                         (300, 256, 3, 4), (300, 128, 4, 2), (400, 512, 2, 4), (250, 256, 8, 1),
                                         (256, 128, 2, 2), (513, 128, 2, 3), (1100, 128, 1, 8)])
def test_prefill_attention(cuda, width, d, b, h):
    """Causal attention over whole contexts (src/omniasr_trt/decode.py:163-164) against the oracle's verify attention
    with query p of a context over keys [0, p]: cache rows addressed through slots, widths that are not multiples
    of the query block (192 queries at head dims 128 and 256, 96 at 512) or of the 32-key tile; heads x contexts a
    multiple of 8 (the XCD-ordered workgroup map) or not (the plain one); at head dim 128 also widths past one
    block and up to six blocks."""
    g = gen(60 + width)
    rows, cap = 5, max(448, -(-width // 64) * 64)
    kc = torch.randn(rows, h, cap, d, generator=g).to(torch.bfloat16)
    vc = torch.randn(rows, h, cap, d, generator=g).to(torch.bfloat16)
    q = torch.randn(b * width, h, d, generator=g).to(torch.bfloat16)
    slots = torch.tensor([4, 0, 2, 1, 3, 0, 4, 2])[:b]
    say(f"prefill attention width={width} d={d} contexts={b} heads={h}")
    out = kernels.prefill_attention(q.to(cuda), kc.to(cuda), vc.to(cuda), slots.to(cuda), width, d ** -0.5)
    torch.cuda.synchronize()
    sl = slots.numpy()
    want = ov.verify_attention(npf(q), npf(kc)[sl], npf(vc)[sl], np.ones(b, np.int64), width, d ** -0.5)
    np.testing.assert_allclose(npf(out), want, atol=BF16_TOL[0], rtol=BF16_TOL[1])


def test_prefill_attention_rejects_bad_shapes(cuda):
    q = torch.zeros(2 * 8, 2, 128, dtype=torch.bfloat16, device=cuda)
    kc = torch.zeros(2, 2, 8, 128, dtype=torch.bfloat16, device=cuda)
    slots = torch.arange(2, device=cuda)
    with pytest.raises(ValueError):  # more positions than the cache holds
        kernels.prefill_attention(q.view(2 * 8, 2, 128)[:16], kc[:, :, :4], kc[:, :, :4], slots, 8, 0.1)
    with pytest.raises(RuntimeError):  # head dim 64: not covered by the kernel
        kernels.prefill_attention(q[..., :64].contiguous(), kc[..., :64].contiguous(), kc[..., :64].contiguous(),
                                  slots, 8, 0.1)


@pytest.mark.parametrize("t", [1, 5, 9])
@pytest.mark.parametrize("d", [16, 512])
def test_verify_attention_f32(cuda, t, d):
    lengths = torch.tensor([600, 257, 1, 0])
    _attn_case(cuda, torch.float32, 4, 8 if d == 512 else 2, d, t, 700, lengths, 640, 4, F32_TOL)


@pytest.mark.parametrize("t", [1, 3, 5, 9])
def test_verify_attention_config3(cuda, t):
    """Config 3: 8 rows, 32 heads x 128, bf16, ragged lengths U[750, 2400], draft 0/2/4/8."""
    g = gen(1003)
    lengths = torch.randint(750, 2401, (8,), generator=g)
    keys = -(-(int(lengths.max()) + t) // 256) * 256
    _attn_case(cuda, torch.bfloat16, 8, 32, 128, t, keys, lengths, keys, 1003, BF16_TOL)


@pytest.mark.parametrize("t", [1, 5, 9, 11, 12, 16])
def test_verify_attention_workgroup_and_split_k(cuda, t):
    """8 rows x 32 heads: the halves kernel (T <= 11) and split-K on the same inputs, both against the oracle; rows
    shorter than one tile per wave, empty, and ending inside a tile."""
    lengths = torch.tensor([2400, 0, 31, 257, 1023, 7, 1800, 96])
    keys = -(-(int(lengths.max()) + t) // 256) * 256
    a = _attn_case(cuda, torch.bfloat16, 8, 32, 128, t, keys, lengths, keys, 31 + t, BF16_TOL)
    b = _attn_case(cuda, torch.bfloat16, 8, 32, 128, t, keys, lengths, keys, 31 + t, BF16_TOL, split_k=True)
    torch.testing.assert_close(a.float(), b.float(), atol=1e-2, rtol=1e-2)


def test_verify_attention_split_choices_agree(cuda):
    """Every split size and both merge modes give the oracle's result, and the two merge modes agree."""
    lengths = torch.tensor([1500, 3, 700, 64, 0, 1023])
    for dtype, d, tol in ((torch.bfloat16, 128, BF16_TOL), (torch.float32, 16, F32_TOL), (torch.bfloat16, 512, BF16_TOL),
                          (torch.bfloat16, 256, BF16_TOL)):
        for chunk in (64, 128, 320, 1536):
            a = _attn_case(cuda, dtype, 6, 4, d, 5, 1536, lengths, 1536, 7, tol, chunk=chunk, separate=False)
            b = _attn_case(cuda, dtype, 6, 4, d, 5, 1536, lengths, 1536, 7, tol, chunk=chunk, separate=True)
            torch.testing.assert_close(a.float(), b.float(), atol=1e-2 if dtype == torch.bfloat16 else 1e-6, rtol=1e-2)


def test_verify_attention_tickets_left_zero(cuda):
    lengths = torch.tensor([900, 17]).to(cuda)
    q = torch.randn(10, 8, 128, device=cuda, dtype=torch.bfloat16)
    kc = torch.randn(2, 8, 1024, 128, device=cuda, dtype=torch.bfloat16)
    for _ in range(3):
        kernels.draft_attention(q, kc, kc, lengths, 5, 1024, 0.1, chunk=64)
    q4 = torch.randn(10, 2, 512, device=cuda, dtype=torch.bfloat16)  # the wide-head kernel's in-kernel merge
    kc4 = torch.randn(2, 2, 1024, 512, device=cuda, dtype=torch.bfloat16)
    for _ in range(3):
        kernels.draft_attention(q4, kc4, kc4, lengths, 5, 1024, 0.1, chunk=64, separate=False)
    torch.cuda.synchronize()
    assert int(kernels._counters[torch.cuda.current_device()].abs().sum()) == 0


@pytest.mark.parametrize("rows,heads", [(43, 3), (256, 1), (9, 16)])
def test_verify_attention_halves_shapes(cuda, rows, heads):
    """The halves kernel at unit counts it must pair exactly: an odd count (the middle workgroup takes both halves
    of one unit), the most rows it takes (256), a count just above its threshold; ragged and empty rows.  The
    tickets are left zero and a second call gives the same bits."""
    g = gen(rows * 7 + heads)
    t, d, cap = 5, 128, 1100
    lengths = torch.randint(0, 1000, (rows,), generator=g)
    lengths[::7] = 0
    lengths[1::5] = torch.randint(1, 40, (len(lengths[1::5]),), generator=g)
    keys = -(-(int(lengths.max()) + t) // 256) * 256
    a = _attn_case(cuda, torch.bfloat16, rows, heads, d, t, cap, lengths, keys, rows + heads, BF16_TOL)
    torch.cuda.synchronize()
    assert int(kernels._counters[torch.cuda.current_device()].abs().sum()) == 0
    b = _attn_case(cuda, torch.bfloat16, rows, heads, d, t, cap, lengths, keys, rows + heads, BF16_TOL)
    assert torch.equal(a, b)


@pytest.mark.parametrize("rows,heads,d,t", [(8, 8, 512, 5), (1, 8, 512, 9), (64, 2, 512, 1), (8, 4, 256, 5),
                                             (3, 8, 512, 16)])
def test_verify_attention_wide_balanced(cuda, rows, heads, d, t):
    """Wide heads (256 / 512) by default run split-K with a fixed workgroup budget per head dealt to the rows by
    their lengths, merged in the kernel: against the oracle and against plain split-K (forced), with empty rows,
    rows shorter than a tile, one row (every workgroup of a head on it) and the most rows the deal takes (64)."""
    g = gen(rows * 31 + d + t)
    lengths = torch.randint(0, 1200, (rows,), generator=g)
    lengths[::5] = 0
    lengths[1::7] = torch.randint(1, 31, (len(lengths[1::7]),), generator=g)
    keys = -(-(int(lengths.max()) + t) // 256) * 256
    a = _attn_case(cuda, torch.bfloat16, rows, heads, d, t, keys, lengths, keys, rows + d, BF16_TOL)
    b = _attn_case(cuda, torch.bfloat16, rows, heads, d, t, keys, lengths, keys, rows + d, BF16_TOL, split_k=True)
    torch.testing.assert_close(a.float(), b.float(), atol=1e-2, rtol=1e-2)
    torch.cuda.synchronize()
    assert int(kernels._counters[torch.cuda.current_device()].abs().sum()) == 0
    c = _attn_case(cuda, torch.bfloat16, rows, heads, d, t, keys, lengths, keys, rows + d, BF16_TOL)
    assert torch.equal(a, c)  # the deal and the merge order are fixed: the same bits every call


@pytest.mark.parametrize("d,h", [(128, 16), (512, 8)])
def test_verify_attention_maximum_lengths(cuda, d, h):
    """Rows at the decoder's position cap (8188 positions, plus the step's 5 queries: 33 tiles past 8000 keys per
    unit), ragged with empty and one-key rows, on the halves kernel (8 x 16 x 128) and the balanced wide-head kernel
    (8 x 8 x 512); the tickets are left zero."""
    lengths = torch.tensor([8188, 8187, 4000, 1, 0, 8100, 7777, 33])
    t = 5
    keys = -(-(int(lengths.max()) + t) // 256) * 256
    _attn_case(cuda, torch.bfloat16, 8, h, d, t, keys, lengths, keys, 90 + d, BF16_TOL)
    torch.cuda.synchronize()
    assert int(kernels._counters[torch.cuda.current_device()].abs().sum()) == 0


def test_verify_attention_wide_graph_replays(cuda):
    """The real checkpoint's shape (8 rows x 8 heads x 512, T = 5) captured once and replayed with new lengths written
    in place: every replay equals the eager call bit for bit, and the tickets are left zero."""
    g = gen(88)
    b, h, d, t, cap = 8, 8, 512, 5, 2560
    kc = torch.randn(b, h, cap, d, generator=g).to(torch.bfloat16).to(cuda)
    vc = torch.randn(b, h, cap, d, generator=g).to(torch.bfloat16).to(cuda)
    q = torch.randn(b * t, h, d, generator=g).to(torch.bfloat16).to(cuda)
    lengths = torch.randint(750, 2401, (b,), generator=g).to(cuda)
    kernels.draft_attention(q, kc, vc, lengths, t, cap, d ** -0.5)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        graph.capture_begin()
        out = kernels.draft_attention(q, kc, vc, lengths, t, cap, d ** -0.5)
        graph.capture_end()
    torch.cuda.current_stream().wait_stream(s)
    gd = torch.Generator(device=cuda).manual_seed(9)
    for rep in range(4):
        lengths.copy_(torch.randint(0, cap - t, (b,), device=cuda, generator=gd))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager = kernels.draft_attention(q, kc, vc, lengths, t, cap, d ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep
    assert int(kernels._counters[torch.cuda.current_device()].abs().sum()) == 0


@pytest.mark.parametrize("split_k", [False, True])
def test_verify_attention_graph_replays(cuda, split_k):
    """Captured in a HIP graph: every replay equals the eager result bit for bit (both decompositions)."""
    g = gen(8)
    b, h, d, t, cap = 8, 32, 128, 5, 2560
    kc = torch.randn(b, h, cap, d, generator=g).to(torch.bfloat16).to(cuda)
    vc = torch.randn(b, h, cap, d, generator=g).to(torch.bfloat16).to(cuda)
    q = torch.randn(b * t, h, d, generator=g).to(torch.bfloat16).to(cuda)
    lengths = torch.randint(750, 2401, (b,), generator=g).to(cuda)
    eager = kernels.draft_attention(q, kc, vc, lengths, t, cap, d ** -0.5, split_k=split_k)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        kernels.draft_attention(q, kc, vc, lengths, t, cap, d ** -0.5, split_k=split_k)
        graph.capture_begin()
        out = kernels.draft_attention(q, kc, vc, lengths, t, cap, d ** -0.5, split_k=split_k)
        graph.capture_end()
    torch.cuda.current_stream().wait_stream(s)
    for i in range(4):
        say(f"graph replay {i}")
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        kernels.draft_attention(q, kc, vc, lengths, t, cap, d ** -0.5, split_k=split_k)  # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("h,d", [(32, 128), (8, 512)])
def test_verify_attention_merge_under_load(cuda, h, d):
    """The in-kernel merges (the halves kernel's tickets at 8 x 32 x 128, the balanced wide-head kernel's at
    8 x 8 x 512) under sustained concurrent load: 96 launches queued back to back on each of two streams -- the
    workspace entry point on one, the static-scratch entry point on the other, so each merge shares its CUs, L2 and
    HBM with the other stream's waves -- over 8 sets of ragged lengths (empty and one-key rows among them).  Every
    launch equals the first eager result for its lengths bit for bit (a partial read before its writer's stores
    landed would change the bits; a ticket left non-zero would break the next launch's merge), those results match
    the oracle, and the workspace path's tickets are left zero."""
    g = gen(70 + d)
    b, t, cap, reps = 8, 5, 2560, 96
    kc = torch.randn(b, h, cap, d, generator=g).to(torch.bfloat16)
    vc = torch.randn(b, h, cap, d, generator=g).to(torch.bfloat16)
    q = torch.randn(b * t, h, d, generator=g).to(torch.bfloat16)
    sets = [torch.randint(750, 2401, (b,), generator=g) for _ in range(8)]
    sets[1][2], sets[3][0], sets[5][7] = 0, 1, 0
    kd, vd, qd = kc.to(cuda), vc.to(cuda), q.to(cuda)
    lens = [s.to(cuda) for s in sets]
    first = [kernels.draft_attention(qd, kd, vd, ln, t, cap, d ** -0.5) for ln in lens]
    torch.cuda.synchronize()
    for j in (0, 1):  # the oracle on two of the sets (the rest are checked through the first results' bits)
        want = ov.verify_attention(npf(q), npf(kc), npf(vc), sets[j].numpy(), t, d ** -0.5)
        np.testing.assert_allclose(npf(first[j]), want, atol=BF16_TOL[0], rtol=BF16_TOL[1])
    outs_a, outs_b = [], []
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    sa.wait_stream(torch.cuda.current_stream())
    sb.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(sb):
        outs_b = [torch.empty_like(qd) for _ in range(reps)]
    say(f"merge under load: h={h} d={d}, {reps} launches on each of two streams")
    for i in range(reps):
        with torch.cuda.stream(sa):
            outs_a.append(kernels.draft_attention(qd, kd, vd, lens[i % 8], t, cap, d ** -0.5))
        with torch.cuda.stream(sb):
            kernels.verify_attention_static(qd, kd, vd, lens[(i + 3) % 8], t, cap, d ** -0.5, outs_b[i])
    torch.cuda.synchronize()
    for i in range(reps):
        assert torch.equal(outs_a[i], first[i % 8]), f"workspace entry point, launch {i}"
        assert torch.equal(outs_b[i], first[(i + 3) % 8]), f"static entry point, launch {i}"
    assert int(kernels._counters[torch.cuda.current_device()].abs().sum()) == 0


# ---------------------------------------------------------------------------------------------- argmax + accept

def _done_state(cuda, b, t, cap=64):
    """State for which acceptance changes nothing (every row finished): only the argmaxes are observed."""
    z = torch.zeros(b, device=cuda, dtype=torch.long)
    return dict(tokens=torch.zeros(b, t, device=cuda, dtype=torch.long),
                out=torch.ones(b, cap, device=cuda, dtype=torch.int32), tok=z.clone(), last=z.clone(),
                done=torch.ones(b, device=cuda, dtype=torch.bool))


ARGMAX_MISMATCH_BOUND = 1e-3  # of all rows: kernel vs PyTorch's GPU op, lse-fragile rows included


def test_argmax_matches_torch_on_the_gpu(cuda):
    """Against PyTorch's own ``F.log_softmax(bf16).argmax`` on the same device, over 4000 rows of N(0, 1) and of
    N(0, 3) logits [40, 10288] (the drafted step's shape): the kernel equals the oracle and PyTorch on every row
    except those whose result hinges on the last bits of the log-sum-exp (flagged by the oracle), and the rows where
    it differs from PyTorch -- fragile ones included -- are counted and stay below ARGMAX_MISMATCH_BOUND."""
    g = gen(1001)
    for scale in (1.0, 3.0):
        fragile_total = mismatches = rows = 0
        for batch in range(100):
            x = (torch.randn(40, 10288, generator=g) * scale).to(torch.bfloat16)
            xd = x.to(cuda)
            st = _done_state(cuda, 8, 5)
            got = kernels.greedy_accept(xd, st["tokens"], st["out"], st["tok"], st["last"], st["done"], None, None,
                                        None, 8188, 2).view(-1).cpu().numpy()
            want = F.log_softmax(xd, -1).argmax(-1).cpu().numpy()
            fragile = ov.argmax_is_fragile(npf(x), "bf16")
            oracle = ov.log_softmax_argmax(npf(x), "bf16")
            assert not ((got != want) & ~fragile).any(), batch
            assert not ((got != oracle) & ~fragile).any(), batch
            fragile_total += int(fragile.sum())
            mismatches += int((got != want).sum())
            rows += x.size(0)
        say(f"argmax N(0, {scale:g}): {rows} rows, {fragile_total} lse-fragile, {mismatches} differ from PyTorch's GPU "
            f"op")
        assert mismatches <= ARGMAX_MISMATCH_BOUND * rows


@pytest.mark.parametrize("v", [12, 10288, 10291])
def test_argmax_fp32_and_odd_vocab(cuda, v):
    g = gen(9)
    x = torch.randn(15, v, generator=g)
    for dtype in (torch.float32, torch.bfloat16):  # odd vocabularies: rows off 16-byte alignment
        xd = x.to(dtype).to(cuda)
        st = _done_state(cuda, 3, 5)
        got = kernels.greedy_accept(xd, st["tokens"], st["out"], st["tok"], st["last"], st["done"], None, None, None,
                                    8188, 2).view(-1).cpu().numpy()
        want = F.log_softmax(xd, -1).argmax(-1).cpu().numpy()
        fragile = ov.argmax_is_fragile(npf(x.to(dtype)), "bf16" if dtype == torch.bfloat16 else "f32")
        assert not ((got != want) & ~fragile).any()


@pytest.mark.parametrize("v,t", [(32768, 2), (32776, 2), (10288, 64)])
def test_argmax_launch_boundaries(cuda, v, t):
    """The row-argmax launch up to 16 chunks per thread (32768 bf16 entries), the one-workgroup-per-slot launch just
    past it, and the most tokens per row (64): against PyTorch on every row the oracle does not flag."""
    g = gen(v + t)
    b = 3
    x = torch.randn(b * t, v, generator=g).to(torch.bfloat16)
    xd = x.to(cuda)
    st = _done_state(cuda, b, t)
    got = kernels.greedy_accept(xd, st["tokens"], st["out"], st["tok"], st["last"], st["done"], None, None, None,
                                8188, 2).view(-1).cpu().numpy()
    want = F.log_softmax(xd, -1).argmax(-1).cpu().numpy()
    fragile = ov.argmax_is_fragile(npf(x), "bf16")
    assert not ((got != want) & ~fragile).any()


def test_accept_golden_vectors(cuda):
    """The reference's own ``_accept`` outputs (Triton interpreter) on 24 states, through ``omni_accept``."""
    z = np.load(GOLD / "accept_golden.npz")
    for c in range(int(z["cases"])):
        p = f"c{c}_"
        d = {k: torch.from_numpy(z[p + k].copy()).to(cuda) for k in
             ("tokens", "nxt", "out", "tok", "last", "done", "draft_next", "start", "use_draft")}
        kernels.accept(d["tokens"], d["nxt"], d["out"], d["tok"], d["last"], d["done"], d["draft_next"], d["start"],
                       d["use_draft"], int(z[p + "limit"]), int(z[p + "eos"]))
        for name in ("out", "tok", "last", "done", "draft_next"):
            np.testing.assert_array_equal(d[name].cpu().numpy(), z[p + name + "_after"], err_msg=f"case {c} {name}")


def _greedy_accept_no_nxt(x, tokens, out, tok, last, done, dn, start, use, limit, eos):
    """``omni_greedy_accept`` with no argmax output (``nxt`` NULL): the one-launch kernel that argmaxes and accepts
    each slot in one workgroup."""
    b, t = tokens.shape
    lib = kernels._lib.load()
    st = lib.omni_greedy_accept(x.data_ptr(), x.stride(0), x.size(1), 1, tokens.data_ptr(), None,
                                out.data_ptr(), out.stride(0), out.size(1), tok.data_ptr(), last.data_ptr(),
                                done.data_ptr(), dn.data_ptr(), start.data_ptr(), use.data_ptr(), b, t, limit, eos,
                                torch.cuda.current_stream().cuda_stream)
    assert st == 0, st


@pytest.mark.parametrize("path,v", [("rows", 10288), ("slot", 10288), ("slot", 40000)])
def test_greedy_accept_state_vs_oracle(cuda, path, v):
    """Logits with planted argmaxes that confirm 0..k drafts, EOS and the limit: the state after the kernel equals
    the oracle's acceptance of the oracle's argmaxes.  ``rows``: the row-argmax launch then the acceptance (the
    argmaxes are returned); ``slot``: one workgroup per slot (no argmax output at 10288, and the path a
    vocabulary past 32768 bf16 entries takes)."""
    g = gen(10)
    rng = np.random.default_rng(10)
    for t in (1, 2, 5, 9):
        b, cap = 8, 512
        x = torch.randn(b * t, v, generator=g)
        tokens = torch.randint(3, v, (b, t), generator=g)
        for r in range(b):  # plant: the argmax after fed token j is fed token j+1 for the first `ok` positions
            ok = int(rng.integers(0, t + 1))
            for j in range(t):
                want = int(tokens[r, j + 1]) if (j < ok and j + 1 < t) else int(rng.integers(3, v))
                if r == 5 and j == 1:
                    want = 2  # EOS
                x[r * t + j, want] = x[r * t + j].max() + 2.0
        x = x.to(torch.bfloat16)
        last = torch.from_numpy(rng.integers(0, cap - 20, b))
        last[6] = 58  # the limit (60) inside the step
        done = torch.from_numpy(rng.random(b) < 0.2)
        out = torch.ones(b, cap, dtype=torch.int32)
        tok = tokens[:, 0].clone()
        dn = torch.from_numpy(rng.integers(0, 900, b))
        start = torch.from_numpy(rng.integers(0, 900, b))
        use = torch.from_numpy(rng.random(b) < 0.5)
        o = [a.numpy().copy() for a in (out, tok, last, done, dn)]
        nxt_o = ov.log_softmax_argmax(npf(x), "bf16").reshape(b, t)
        ov.accept(tokens.numpy(), nxt_o, o[0], o[1], o[2], o[3], o[4], start.numpy(), use.numpy(), 60, 2)
        d = [a.to(cuda) for a in (out, tok, last, done, dn)]
        say(f"greedy_accept {path} v={v} t={t}")
        if path == "slot" and v == 10288:
            _greedy_accept_no_nxt(x.to(cuda), tokens.to(cuda), *d, start.to(cuda), use.to(cuda), 60, 2)
        else:
            nxt = kernels.greedy_accept(x.to(cuda), tokens.to(cuda), d[0], d[1], d[2], d[3], d[4], start.to(cuda),
                                        use.to(cuda), 60, 2)
            np.testing.assert_array_equal(nxt.cpu().numpy(), nxt_o)
        for got, want in zip(d, o):
            np.testing.assert_array_equal(got.cpu().numpy(), want)


def test_config1_verify_step(cuda):
    """Config 1: one row, 5 queries (1 + 4 drafts), 32 x 128, 1024 prior keys; logits [5, 10288] N(0,1) with the
    argmax planted on the first 2 drafts -> 3 tokens accepted, the cache length rolled forward by 3."""
    g = gen(1001)
    h, d, t, n = 32, 128, 5, 1024
    kc = torch.randn(1, h, 1280, d, generator=g).to(torch.bfloat16)
    vc = torch.randn(1, h, 1280, d, generator=g).to(torch.bfloat16)
    q = torch.randn(t, h, d, generator=g).to(torch.bfloat16)
    out = kernels.draft_attention(q.to(cuda), kc.to(cuda), vc.to(cuda), torch.tensor([n + 1]).to(cuda), t, 1280,
                                  d ** -0.5)
    want = ov.verify_attention(npf(q), npf(kc), npf(vc), np.array([n + 1]), t, d ** -0.5)
    np.testing.assert_allclose(npf(out), want, atol=2e-2, rtol=1e-2)
    drafts = torch.randint(3, 10288, (4,), generator=g)
    x = torch.randn(t, 10288, generator=g)
    x[0, drafts[0]] = x[0].max() + 1.0
    x[1, drafts[1]] = x[1].max() + 1.0
    x[2, int(drafts[2])] = x[2].min() - 1.0  # the row-2 maximum is not d3
    x = x.to(torch.bfloat16)
    tokens = torch.cat([torch.tensor([7]), drafts])[None].to(cuda)
    st = dict(out=torch.ones(1, 2048, dtype=torch.int32, device=cuda), tok=torch.tensor([7], device=cuda),
              last=torch.tensor([n], device=cuda), done=torch.zeros(1, dtype=torch.bool, device=cuda))
    nxt = kernels.greedy_accept(x.to(cuda), tokens, st["out"], st["tok"], st["last"], st["done"], None, None, None,
                                8188, 2)
    assert nxt[0, 0] == drafts[0] and nxt[0, 1] == drafts[1] and nxt[0, 2] != drafts[2]
    assert int(st["last"]) == n + 3 and not bool(st["done"])
    assert st["out"][0, n + 1: n + 4].tolist() == [int(drafts[0]), int(drafts[1]), int(nxt[0, 2])]


# ---------------------------------------------------------------------------------------------- propose

def test_propose_golden_vectors(cuda):
    z = np.load(GOLD / "propose_golden.npz")
    for tr in range(int(z["trials"])):
        p = f"t{tr}_"
        a = {k: torch.from_numpy(z[p + k].copy()).to(cuda) for k in ("out", "draft", "draft_len", "last", "first",
                                                                      "next")}
        start = torch.empty(a["last"].numel(), dtype=torch.long, device=cuda)
        prop, use = kernels.propose(a["out"], a["draft"], a["draft_len"], a["last"], a["first"], a["next"], start,
                                    int(z[p + "k"]), NGRAM, BEHIND, AHEAD, REACH, SELF_WINDOW, SELF_MIN)
        np.testing.assert_array_equal(prop.cpu().numpy(), z[p + "prop"], err_msg=f"trial {tr}")
        np.testing.assert_array_equal(use.cpu().numpy(), z[p + "use_draft"], err_msg=f"trial {tr}")
        np.testing.assert_array_equal(start.cpu().numpy(), z[p + "start"], err_msg=f"trial {tr}")


@pytest.mark.parametrize("k", [1, 4, 7])
def test_propose_vs_oracle(cuda, k):
    """The reference test's generator (src tests/test_spec.py:201-226), 20 trials, vocabularies of 4-8."""
    g = gen(30 + k)
    for trial in range(20):
        vocab = 4 + trial % 5
        b, cap = 8, 2048
        out = torch.randint(3, vocab, (b, cap), dtype=torch.int32, generator=g)
        first = torch.randint(0, 600, (b,), generator=g)
        last = first + torch.randint(0, 1400, (b,), generator=g)
        last[0] = first[0]
        out[torch.arange(cap)[None, :] < first[:, None]] = 1
        draft = torch.randint(3, vocab, (b, 1024), dtype=torch.int32, generator=g)
        dlen = torch.randint(0, 1025, (b,), generator=g)
        dlen[1] = 0
        draft[torch.arange(1024)[None, :] >= dlen[:, None]] = -1
        nxt = (torch.rand(b, generator=g) * (dlen + 8)).long()
        want = ov.propose(out.numpy(), draft.numpy(), dlen.numpy(), last.numpy(), first.numpy(), nxt.numpy(), k,
                          NGRAM, BEHIND, AHEAD, REACH, 256, 256, SELF_MIN)
        start = torch.empty(b, dtype=torch.long, device=cuda)
        prop, use = kernels.propose(out.to(cuda), draft.to(cuda), dlen.to(cuda), last.to(cuda), first.to(cuda),
                                    nxt.to(cuda), start, k, NGRAM, BEHIND, AHEAD, REACH, SELF_WINDOW, SELF_MIN)
        np.testing.assert_array_equal(prop.cpu().numpy(), want[0], err_msg=f"trial {trial}")
        np.testing.assert_array_equal(use.cpu().numpy(), want[1], err_msg=f"trial {trial}")
        np.testing.assert_array_equal(start.cpu().numpy(), want[2], err_msg=f"trial {trial}")


def test_spec_prepare_vs_oracle(cuda):
    g = gen(12)
    b, cap, k = 8, 2048, 4
    out = torch.randint(3, 6, (b, cap), dtype=torch.int32, generator=g)
    first = torch.randint(0, 600, (b,), generator=g)
    last = first + torch.randint(0, 1400, (b,), generator=g)
    last[2] = cap - 2  # positions past the cache end are clamped
    draft = torch.randint(3, 6, (b, 1024), dtype=torch.int32, generator=g)
    dlen = torch.randint(0, 1025, (b,), generator=g)
    nxt = (torch.rand(b, generator=g) * (dlen + 8)).long()
    tok = torch.randint(3, 6, (b,), generator=g)
    done = torch.tensor([False, True, False, False, True, False, False, False])
    want = ov.spec_prepare(out.numpy(), draft.numpy(), dlen.numpy(), last.numpy(), first.numpy(), nxt.numpy(),
                           tok.numpy(), done.numpy(), cap, k, NGRAM, BEHIND, AHEAD, REACH, 256, 256, SELF_MIN)
    start = torch.empty(b, dtype=torch.long, device=cuda)
    got = kernels.spec_prepare(out.to(cuda), draft.to(cuda), dlen.to(cuda), last.to(cuda), first.to(cuda),
                               nxt.to(cuda), start, tok.to(cuda), done.to(cuda), cap, k, NGRAM, BEHIND, AHEAD, REACH,
                               SELF_WINDOW, SELF_MIN)
    for x, y in zip(got, want[:5]):
        np.testing.assert_array_equal(x.cpu().numpy().reshape(y.shape), y)
    np.testing.assert_array_equal(start.cpu().numpy(), want[5])

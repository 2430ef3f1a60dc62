"""Beam search on the HIP kernels: ``beam_attention`` against the oracle (fp64), and ``BeamDecoder`` against the
reference-order beam loop on small random fp32 models (src tests/test_beam.py, tests/test_kernels.py:98-147)."""

import sys

import numpy as np
import pytest
import torch

from oracle import reference as oref
from oracle import verify as ov
from omniasr_trt_amd import beam, kernels, llm
from omniasr_trt_amd.beam import BeamDecoder
from omniasr_trt_amd.decode import GreedyDecoder

from test_decode_gpu import contexts, gpu_pair

pytestmark = pytest.mark.gpu

BF16_TOL = (2e-2, 1e-2)
F32_TOL = (1e-4, 1e-4)


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def npf(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def _beam_inputs(dtype, groups, beams, h, d, cap, gcap, ctx_len, gen_len, seed):
    g = torch.Generator().manual_seed(seed)
    rows = groups * beams
    kc = torch.randn(groups + 1, h, cap, d, generator=g).to(dtype)
    vc = torch.randn(groups + 1, h, cap, d, generator=g).to(dtype)
    kg = torch.randn(rows + 2, h, gcap, d, generator=g).to(dtype)
    vg = torch.randn(rows + 2, h, gcap, d, generator=g).to(dtype)
    q = torch.randn(rows, h, d, generator=g).to(dtype)
    ptr = torch.randint(0, rows + 2, (rows, gcap), generator=g, dtype=torch.int32)
    return q, kc, vc, kg, vg, ptr, torch.as_tensor(ctx_len), torch.as_tensor(gen_len)


def _beam_case(cuda, dtype, groups, beams, h, d, cap, gcap, ctx_len, gen_len, ctx_keys, seed, tol, chunk=0):
    q, kc, vc, kg, vg, ptr, cl, gl = _beam_inputs(dtype, groups, beams, h, d, cap, gcap, ctx_len, gen_len, seed)
    say(f"beam attention dtype={dtype} groups={groups} beams={beams} h={h} d={d} ctx={cl.tolist()[:8]} "
        f"gen_max={int(gl.max())} chunk={chunk}")
    out = kernels.beam_attention(q.to(cuda), kc.to(cuda), vc.to(cuda), cl.to(cuda), kg.to(cuda), vg.to(cuda),
                                 ptr.to(cuda), gl.to(cuda), beams, ctx_keys, d ** -0.5, chunk=chunk)
    torch.cuda.synchronize()
    want = ov.beam_attention(npf(q), npf(kc), npf(vc), cl.numpy(), npf(kg), npf(vg), ptr.numpy(), gl.numpy(), beams,
                             d ** -0.5)
    np.testing.assert_allclose(npf(out), want, atol=tol[0], rtol=tol[1])
    return out


@pytest.mark.parametrize("beams", [1, 3, 5])
@pytest.mark.parametrize("d", [128, 64, 256, 512])
def test_beam_attention_bf16(cuda, beams, d):
    """The reference's case (tests/test_kernels.py:98-126): a finished input reads nothing, ragged generated
    lengths, pointers anywhere in the generated rows."""
    groups = 4
    gen_len = torch.randint(0, 300, (groups * beams,), generator=torch.Generator().manual_seed(beams))
    gen_len[-beams:] = 0
    out = _beam_case(cuda, torch.bfloat16, groups, beams, 8, d, 600, 300, [600, 333, 1, 0], gen_len, 640, 9,
                     BF16_TOL)
    assert torch.all(out[-beams:] == 0)


@pytest.mark.parametrize("beams", [1, 4])
@pytest.mark.parametrize("d", [16, 512])
def test_beam_attention_f32(cuda, beams, d):
    gen_len = torch.randint(0, 70, (3 * beams,), generator=torch.Generator().manual_seed(d))
    _beam_case(cuda, torch.float32, 3, beams, 2, d, 300, 70, [300, 65, 0], gen_len, 320, 10, F32_TOL)


@pytest.mark.parametrize("beams", [1, 3, 5])
def test_beam_attention_f32_reference_case(cuda, beams):
    """The reference's fp32 case (tests/test_kernels.py:98-126) at its shape: 4 inputs x 8 heads x 512, contexts
    [600, 333, 1, 0] in a cache of 600, 300 generated positions, the last input finished, within its 1e-4."""
    gen_len = torch.randint(0, 300, (4 * beams,), generator=torch.Generator().manual_seed(20 + beams))
    gen_len[-beams:] = 0
    out = _beam_case(cuda, torch.float32, 4, beams, 8, 512, 600, 300, [600, 333, 1, 0], gen_len, 640, 21, F32_TOL)
    assert torch.all(out[-beams:] == 0)


def test_beam_attention_config5(cuda):
    """Config 5 (beam variant): 8 inputs x 5 beams, 32 heads x 128, contexts U[750, 2400], 1-160 generated keys;
    several split sizes."""
    g = torch.Generator().manual_seed(55)
    ctx_len = torch.randint(750, 2401, (8,), generator=g)
    gen_len = torch.randint(1, 161, (40,), generator=g)
    keys = -(-int(ctx_len.max()) // 256) * 256
    for chunk in (0, 64, 256):
        _beam_case(cuda, torch.bfloat16, 8, 5, 32, 128, keys, 256, ctx_len, gen_len, keys, 56, BF16_TOL, chunk=chunk)


@pytest.mark.parametrize("beams", [3, 5, 11, 12])
def test_beam_attention_context_halves(cuda, beams):
    """8 inputs x 32 heads x 128: the halves kernel with each unit's generated keys as tiles after its context (beams
    <= 11; 12 takes split-K and the generated keys' own launch) -- finished inputs (no context, no generated keys), a
    context shorter than a tile, generated keys only."""
    g = torch.Generator().manual_seed(70 + beams)
    ctx_len = torch.tensor([2300, 0, 17, 1500, 0, 640, 999, 33])
    gen_len = torch.randint(0, 97, (8 * beams,), generator=g)
    gen_len[beams: 2 * beams] = 0  # input 1 finished
    keys = 2304
    _beam_case(cuda, torch.bfloat16, 8, beams, 32, 128, keys, 96, ctx_len, gen_len, keys, 71, BF16_TOL)


def test_beam_attention_generated_tiles_edges(cuda):
    """The halves kernel with the generated keys as tiles of its deal, at an odd unit count (43 inputs x 3 heads: the
    middle workgroup takes both halves of one unit): empty contexts whose generated keys are then all of the unit's
    tiles (both halves), beams with no generated keys beside beams with many, generated lists longer than the
    context, finished inputs; the tickets are left zero and a second call gives the same bits."""
    g = torch.Generator().manual_seed(123)
    groups, beams = 43, 3
    ctx_len = torch.randint(0, 400, (groups,), generator=g)
    ctx_len[::6] = 0
    gen_len = torch.randint(0, 201, (groups * beams,), generator=g)
    gen_len[1::4] = 0
    gen_len[6:9] = 0  # input 2: nothing generated
    ctx_len[2] = 0  # and no context: a finished input
    keys = 512
    a = _beam_case(cuda, torch.bfloat16, groups, beams, 3, 128, keys, 200, ctx_len, gen_len, keys, 124, BF16_TOL)
    assert torch.all(a[6:9] == 0)
    torch.cuda.synchronize()
    assert int(kernels._counters[torch.cuda.current_device()].abs().sum()) == 0
    b = _beam_case(cuda, torch.bfloat16, groups, beams, 3, 128, keys, 200, ctx_len, gen_len, keys, 124, BF16_TOL)
    assert torch.equal(a, b)


@pytest.mark.parametrize("h,d", [(16, 128), (8, 512)])
def test_beam_attention_long_generation(cuda, h, d):
    """8 inputs x 5 beams with a generated cache of 1024 positions: more generated positions per unit than the
    context kernels' tables hold (the halves kernel at 16 heads x 128, the balanced wide-head kernel at 8 x 512), so
    the generated keys run in their own launch and the context launch merges its partial; lengths up to the
    capacity."""
    g = torch.Generator().manual_seed(125)
    ctx_len = torch.tensor([1500, 0, 333, 2000, 1, 900, 64, 1200])
    gen_len = torch.randint(0, 1025, (40,), generator=g)
    gen_len[:5] = torch.tensor([1024, 1023, 0, 1, 512])
    gen_len[5:10] = 0  # input 1 finished
    keys = 2048
    out = _beam_case(cuda, torch.bfloat16, 8, 5, h, d, keys, 1024, ctx_len, gen_len, keys, 126, BF16_TOL)
    assert torch.all(out[5:10] == 0)
    torch.cuda.synchronize()
    assert int(kernels._counters[torch.cuda.current_device()].abs().sum()) == 0


def _shared_pointers(groups, beams, gcap, rows, seed, share=0.85):
    """Pointers like a beam search's: at each position the beams of a group mostly reach one row (a shared
    history), sometimes their own, and a few out of range (clamped by the kernels)."""
    g = np.random.default_rng(seed)
    ptr = np.zeros((groups * beams, gcap), dtype=np.int32)
    for grp in range(groups):
        common = g.integers(0, rows, gcap)
        for e in range(beams):
            own = g.integers(0, rows, gcap)
            ptr[grp * beams + e] = np.where(g.random(gcap) < share, common, own)
    ptr[0, :3] = [-4, rows + 7, rows - 1]
    return torch.as_tensor(ptr)


def _list_reference(ptr, gen_len, groups, beams, gcap, rows, g_row, g_pos):
    """Each group's distinct (row, position) keys: by position, then by the first beam that reaches the key; the
    byte offset (row * g_row + position * g_pos) * 2 and the mask of the beams that see it."""
    out = []
    for grp in range(groups):
        n = [int(np.clip(gen_len[grp * beams + e], 0, gcap)) for e in range(beams)]
        offs, masks = [], []
        for j in range(max(n)):
            src = [int(np.clip(ptr[grp * beams + e, j], 0, rows - 1)) if j < n[e] else -1 for e in range(beams)]
            for e in range(beams):
                if src[e] < 0 or src[e] in src[:e]:
                    continue
                offs.append((src[e] * g_row + j * g_pos) * 2)
                masks.append(sum(1 << e2 for e2 in range(beams) if src[e2] == src[e]))
        out.append((offs, masks))
    return out


@pytest.mark.parametrize("beams,d", [(5, 128), (16, 512), (1, 128)])
def test_beam_gen_list(cuda, beams, d):
    """kernels.beam_gen_list: every group's distinct generated keys with the beams that see each, in position
    order, against the list restated in Python -- ragged and empty generations, clamped pointers, 16 beams."""
    groups, gcap, h = 6, 160, 2
    rows = groups * beams
    kg = torch.empty(rows + 2, h, gcap, d, dtype=torch.bfloat16, device=cuda)
    ptr = _shared_pointers(groups, beams, gcap, rows + 2, 7 + beams)
    gen_len = torch.randint(0, gcap + 1, (rows,), generator=torch.Generator().manual_seed(beams))
    gen_len[beams: 2 * beams] = 0
    gen_len[0] = gcap
    lst = kernels.GenList(groups, beams, gcap, cuda)
    kernels.beam_gen_list(lst, ptr.to(cuda), gen_len.to(cuda), kg, groups)
    torch.cuda.synchronize()
    want = _list_reference(ptr.numpy(), gen_len.numpy(), groups, beams, gcap, rows + 2, kg.stride(0), kg.stride(2))
    offs = lst.offsets.cpu().numpy().view(np.uint32)
    masks = lst.masks.cpu().numpy().view(np.uint16)
    counts = lst.counts.cpu().numpy()
    for grp, (w_off, w_mask) in enumerate(want):
        assert counts[grp] == len(w_off), grp
        np.testing.assert_array_equal(offs[grp, :counts[grp]], np.array(w_off, dtype=np.uint32), err_msg=str(grp))
        np.testing.assert_array_equal(masks[grp, :counts[grp]], np.array(w_mask, dtype=np.uint16), err_msg=str(grp))
    total = int(sum(min(int(x), gcap) for x in gen_len))
    say(f"beam_gen_list beams={beams}: {total} generated keys, {int(counts.sum())} distinct")
    if beams > 1:
        assert counts.sum() < total / 2  # the beams share most keys


@pytest.mark.parametrize("h,d,beams,gcap", [(32, 128, 5, 128), (8, 512, 5, 128), (32, 128, 11, 372),
                                             (8, 512, 16, 256), (8, 512, 16, 257)])
def test_beam_attention_with_gen_list(cuda, h, d, beams, gcap):
    """Both context kernels with the step's list of distinct generated keys: against the oracle and against the
    same call without the list, pointers shared like a beam search's, ragged generations, a finished input, an input
    with generated keys only; then captured in a graph with the list's build and replayed with new pointers and
    lengths, every replay equal to the eager calls bit for bit; the tickets are left zero.  The halves kernel's most
    beams (11), a wide-head table of exactly 4096 keys (16 beams x 256), and one key more, where the generated keys
    go to their own launch and the list is not read."""
    groups = 8
    rows = groups * beams
    say(f"gen list h={h} d={d} beams={beams} gen_cap={gcap}")
    ctx_len = torch.tensor([2000, 0, 333, 1500, 0, 900, 64, 1200])
    gen_len = torch.randint(0, gcap + 1, (rows,), generator=torch.Generator().manual_seed(h + beams))
    gen_len[beams: 2 * beams] = 0  # input 1 finished
    q, kc, vc, kg, vg, _, cl, gl = _beam_inputs(torch.bfloat16, groups, beams, h, d, 2048, gcap, ctx_len, gen_len, 31)
    ptr = _shared_pointers(groups, beams, gcap, rows + 2, 32)
    want = ov.beam_attention(npf(q), npf(kc), npf(vc), cl.numpy(), npf(kg), npf(vg), ptr.numpy(), gl.numpy(), beams,
                             d ** -0.5)
    q, kc, vc, kg, vg, ptr, cl, gl = (t.to(cuda) for t in (q, kc, vc, kg, vg, ptr, cl, gl))
    lst = kernels.GenList(groups, beams, gcap, cuda)
    kernels.beam_gen_list(lst, ptr, gl, kg, groups)
    got = kernels.beam_attention(q, kc, vc, cl, kg, vg, ptr, gl, beams, 2048, d ** -0.5, gen_list=lst)
    plain = kernels.beam_attention(q, kc, vc, cl, kg, vg, ptr, gl, beams, 2048, d ** -0.5)
    torch.cuda.synchronize()
    np.testing.assert_allclose(npf(got), want, atol=BF16_TOL[0], rtol=BF16_TOL[1])
    torch.testing.assert_close(got.float(), plain.float(), atol=1e-2, rtol=1e-2)
    assert torch.all(got[beams: 2 * beams] == 0)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        graph.capture_begin()
        kernels.beam_gen_list(lst, ptr, gl, kg, groups)
        out = kernels.beam_attention(q, kc, vc, cl, kg, vg, ptr, gl, beams, 2048, d ** -0.5, gen_list=lst)
        graph.capture_end()
    torch.cuda.current_stream().wait_stream(stream)
    for rep in range(3):
        ptr.copy_(_shared_pointers(groups, beams, gcap, rows + 2, 40 + rep).to(cuda))
        gl.copy_(torch.randint(0, gcap + 1, (rows,), generator=torch.Generator().manual_seed(50 + rep)).to(cuda))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        kernels.beam_gen_list(lst, ptr, gl, kg, groups)
        eager = kernels.beam_attention(q, kc, vc, cl, kg, vg, ptr, gl, beams, 2048, d ** -0.5, gen_list=lst)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep
    assert int(kernels._counters[torch.cuda.current_device()].abs().sum()) == 0


@pytest.mark.parametrize("beams", [1, 5, 16])
def test_beam_attention_wide_balanced(cuda, beams):
    """8 inputs x 8 heads x 512 (the real checkpoint's shape): the balanced wide-head kernel with each input's
    generated keys as tiles after its context, dealt with them over the (input, head)'s workgroups, whose last one
    merges the splits -- finished inputs (no context, no generated keys), a context shorter than a tile, generated
    keys only, up to 16 beams."""
    g = torch.Generator().manual_seed(90 + beams)
    ctx_len = torch.tensor([2300, 0, 17, 1500, 0, 640, 999, 33])
    gen_len = torch.randint(0, 97, (8 * beams,), generator=g)
    gen_len[beams: 2 * beams] = 0  # input 1 finished
    out = _beam_case(cuda, torch.bfloat16, 8, beams, 8, 512, 2304, 96, ctx_len, gen_len, 2304, 91, BF16_TOL)
    assert torch.all(out[beams: 2 * beams] == 0)


@pytest.mark.parametrize("d,h", [(128, 32), (512, 8)])
def test_beam_attention_maximum_lengths(cuda, d, h):
    """Contexts at the position cap (8188 keys), 5 beams, up to 300 generated keys, a finished input: the halves
    kernel (8 inputs x 32 heads x 128) and the balanced wide-head kernel (8 x 8 x 512)."""
    g = torch.Generator().manual_seed(95 + d)
    ctx_len = torch.tensor([8188, 8000, 1, 0, 4097, 8187, 33, 7000])
    gen_len = torch.randint(0, 301, (40,), generator=g)
    gen_len[15:20] = 0  # input 3 finished
    keys = -(-8188 // 256) * 256
    out = _beam_case(cuda, torch.bfloat16, 8, 5, h, d, keys, 320, ctx_len, gen_len, keys, 96, BF16_TOL)
    assert torch.all(out[15:20] == 0)


def test_beam_attention_wide_graph_replays(cuda):
    """The balanced wide-head path (4 inputs x 3 beams x 8 heads x 512) captured once and replayed with new lengths
    and pointers; every replay equals the eager call bit for bit (the tickets are left zero between calls)."""
    q, kc, vc, kg, vg, ptr, cl, gl = _beam_inputs(torch.bfloat16, 4, 3, 8, 512, 1024, 64, [1000, 0, 77, 1024],
                                                  [5, 0, 17, 64, 33, 1, 9, 3, 60, 2, 0, 41], 14)
    q, kc, vc, kg, vg, ptr, cl, gl = (t.to(cuda) for t in (q, kc, vc, kg, vg, ptr, cl, gl))
    kernels.beam_attention(q, kc, vc, cl, kg, vg, ptr, gl, 3, 1024, 512 ** -0.5)  # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        graph.capture_begin()
        out = kernels.beam_attention(q, kc, vc, cl, kg, vg, ptr, gl, 3, 1024, 512 ** -0.5)
        graph.capture_end()
    torch.cuda.current_stream().wait_stream(stream)
    g = torch.Generator(device=cuda).manual_seed(4)
    for rep in range(4):
        ptr.copy_(torch.randint(0, 14, ptr.shape, device=cuda, generator=g, dtype=torch.int32))
        gl.copy_(torch.randint(0, 65, gl.shape, device=cuda, generator=g))
        cl.copy_(torch.randint(0, 1025, cl.shape, device=cuda, generator=g))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager = kernels.beam_attention(q, kc, vc, cl, kg, vg, ptr, gl, 3, 1024, 512 ** -0.5)
        assert torch.equal(out, eager), rep


def test_beam_attention_graph_replays(cuda):
    """Captured once, replayed with new pointers and lengths written in place between replays."""
    q, kc, vc, kg, vg, ptr, cl, gl = _beam_inputs(torch.bfloat16, 4, 3, 8, 128, 512, 128, [500, 200, 37, 512],
                                                  [5, 0, 17, 128, 64, 1, 9, 3, 100, 2, 0, 77], 12)
    q, kc, vc, kg, vg, ptr, cl, gl = (t.to(cuda) for t in (q, kc, vc, kg, vg, ptr, cl, gl))
    kernels.beam_attention(q, kc, vc, cl, kg, vg, ptr, gl, 3, 512, 128 ** -0.5)  # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        graph.capture_begin()
        out = kernels.beam_attention(q, kc, vc, cl, kg, vg, ptr, gl, 3, 512, 128 ** -0.5)
        graph.capture_end()
    torch.cuda.current_stream().wait_stream(stream)
    g = torch.Generator(device=cuda).manual_seed(3)
    for rep in range(4):
        ptr.copy_(torch.randint(0, 14, ptr.shape, device=cuda, generator=g, dtype=torch.int32))
        gl.copy_(torch.randint(0, 129, gl.shape, device=cuda, generator=g))
        cl.copy_(torch.randint(0, 513, cl.shape, device=cuda, generator=g))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager = kernels.beam_attention(q, kc, vc, cl, kg, vg, ptr, gl, 3, 512, 128 ** -0.5)
        assert torch.equal(out, eager), rep


def test_beam_attention_halves_graph_replays(cuda):
    """The halves path (8 inputs x 5 beams x 32 heads) captured once and replayed with new lengths and pointers;
    every replay equals the eager call bit for bit (the tickets are left zero between calls)."""
    q, kc, vc, kg, vg, ptr, cl, gl = _beam_inputs(torch.bfloat16, 8, 5, 32, 128, 1024, 64,
                                                  [1000, 0, 512, 77, 1024, 3, 640, 900],
                                                  torch.randint(0, 65, (40,), generator=torch.Generator().manual_seed(5)),
                                                  13)
    q, kc, vc, kg, vg, ptr, cl, gl = (t.to(cuda) for t in (q, kc, vc, kg, vg, ptr, cl, gl))
    kernels.beam_attention(q, kc, vc, cl, kg, vg, ptr, gl, 5, 1024, 128 ** -0.5)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        graph.capture_begin()
        out = kernels.beam_attention(q, kc, vc, cl, kg, vg, ptr, gl, 5, 1024, 128 ** -0.5)
        graph.capture_end()
    torch.cuda.current_stream().wait_stream(stream)
    g = torch.Generator(device=cuda).manual_seed(4)
    for rep in range(4):
        ptr.copy_(torch.randint(0, 42, ptr.shape, device=cuda, generator=g, dtype=torch.int32))
        gl.copy_(torch.randint(0, 65, gl.shape, device=cuda, generator=g))
        cl.copy_(torch.randint(0, 1025, cl.shape, device=cuda, generator=g))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager = kernels.beam_attention(q, kc, vc, cl, kg, vg, ptr, gl, 5, 1024, 128 ** -0.5)
        assert torch.equal(out, eager), rep
    assert int(kernels._counters[torch.cuda.current_device()].abs().sum()) == 0


def test_beam_attention_rejects_bad_shapes(cuda):
    q, kc, vc, kg, vg, ptr, cl, gl = (t.to(cuda) for t in _beam_inputs(torch.bfloat16, 2, 2, 2, 64, 64, 16,
                                                                       [4, 4], [1, 1, 1, 1], 0))
    with pytest.raises(ValueError):
        kernels.beam_attention(q, kc, vc, cl, kg, vg, ptr[:, :8], gl, 2, 64, 0.125)  # fewer pointers than positions
    with pytest.raises(ValueError):
        kernels.beam_attention(q, kc, vc, cl, kg, vg, ptr.long(), gl, 2, 64, 0.125)
    with pytest.raises(kernels._lib.KernelError):
        kernels.beam_attention(q[:2].repeat(9, 1, 1), kc, vc, torch.zeros(1, dtype=torch.long, device=cuda),
                               kg.repeat(5, 1, 1, 1), vg.repeat(5, 1, 1, 1), ptr.repeat(5, 1), gl.repeat(5), 18, 64,
                               0.125)  # 18 beams: more queries than the kernel takes


# ---------------------------------------------------------------------------------------------- the decoder

# A beam search compares sums of log-probabilities across hypotheses: where two offers at the survivors' boundary
# (or two survivors) are closer than the difference between fp32 and fp64 arithmetic, both choices are correct
# roundings of the same search.  The fixtures below are contexts whose oracle run has no such near-tie (every gap
# among the best beams + 1 offers above ROBUST, relative), so the HIP path must give exactly the reference's tokens.
ROBUST = 2e-5


def picked(picks, lengths):
    """Context i of ``contexts(seed, lengths)`` for each (seed, i)."""
    return [contexts(seed, lengths)[i] for seed, i in picks]


def references(ref_dec, ctxs, beams, length_norm, **kw):
    out = []
    for c in ctxs:
        margins = []
        out.append(oref.beam_reference(ref_dec, c, beams, length_norm, margins=margins, **kw))
        assert min(margins) > ROBUST, f"fixture of length {c.size(0)} has a near-tie ({min(margins):.1e})"
    return out


@pytest.mark.parametrize("beams,length_norm", [(2, False), (5, False), (5, True), (3, True)])
def test_beam_decoder_matches_reference_order(cuda, beams, length_norm):
    m, ref_dec = gpu_pair(12)
    ctxs = picked(((5, 2), (13, 0), (13, 1), (11, 3), (9, 4), (6, 2), (10, 1)), (6, 40, 13, 25, 9))
    ref = references(ref_dec, ctxs, beams, length_norm)
    assert len({tuple(r) for r in ref}) > 1
    for graphs in (False, True):
        say(f"beam decoder beams={beams} length_norm={length_norm} graphs={graphs}")
        # fewer groups than inputs: a finished group takes the next input
        dec = BeamDecoder(m, beams=beams, length_norm=length_norm, max_batch=2, sync_every=5, graphs=graphs,
                          reserve=16)
        assert dec.generate([c.cuda() for c in ctxs]) == ref
        assert dec.generate([c.cuda() for c in ctxs[:2]]) == ref[:2]


def test_beam_changes_the_result(cuda):
    """The fixtures are not all decided greedily: beam search picks other texts for some of them."""
    m, ref_dec = gpu_pair(12)
    ctxs = picked(((5, 2), (13, 0), (13, 1), (11, 3)), (6, 40, 13, 25, 9))
    greedy = GreedyDecoder(m, max_batch=2, sync_every=5, reserve=16).generate([c.cuda() for c in ctxs])
    beams = BeamDecoder(m, beams=5, max_batch=2, sync_every=5, reserve=16).generate([c.cuda() for c in ctxs])
    assert beams == references(ref_dec, ctxs, 5, False)
    assert sum(g != b for g, b in zip(greedy, beams)) >= 2


def test_one_beam_is_the_greedy_decoder(cuda):
    m, ref_dec = gpu_pair(11)
    ctxs = [c.cuda() for c in contexts(1, (5, 30, 17))]
    want = GreedyDecoder(m, max_batch=3, sync_every=4, reserve=16).generate(ctxs)
    assert BeamDecoder(m, beams=1, max_batch=2, sync_every=4, reserve=16).generate(ctxs) == want
    assert want == [oref.greedy_reference(ref_dec, c.cpu()) for c in ctxs]


@pytest.mark.parametrize("beams,length_norm", [(3, False), (4, True)])
def test_repetition_stop_lands_on_the_same_step(cuda, monkeypatch, beams, length_norm):
    """EOS logit zeroed (the others are peaked): hypotheses loop until the repetition stop ends them at a checked
    position, which must happen at the step it happens in the reference loop.  Buckets of 32 positions: the
    generated caches grow every few host looks and the context caches when a longer context arrives; the grown
    caches are released at the end of the call."""
    monkeypatch.setattr(beam, "LIMIT", 700)
    monkeypatch.setattr(beam, "KEY_BUCKET", 32)
    m, ref_dec = gpu_pair(15, edit=lambda m: m.final_proj.weight.data[llm.EOS].zero_())
    ctxs = picked(((8, 5), (10, 2), (10, 6), (9, 5), (7, 2), (11, 4)), (5, 60, 140, 151, 30, 99, 20, 120))
    ref = references(ref_dec, ctxs, beams, length_norm, limit=700)
    dec = BeamDecoder(m, beams=beams, length_norm=length_norm, max_batch=3, sync_every=7, reserve=16)
    dec.context_floor = 0
    say(f"repetition stop beams={beams} length_norm={length_norm}")
    assert dec.generate([c.cuda() for c in ctxs]) == ref
    assert dec.stats["repetition_stops"] >= 1
    assert dec.stats["grows"] >= 1 and dec.ccap == dec.gcap == 0
    assert dec.generate([ctxs[0].cuda()]) == ref[:1]


def test_position_cap(cuda, monkeypatch):
    monkeypatch.setattr(beam, "LIMIT", 40)
    m, ref_dec = gpu_pair(23, edit=lambda m: m.final_proj.weight.data[llm.EOS].mul_(0.3))
    ctxs = contexts(24, (5, 30, 39, 41, 12))
    ref = references(ref_dec, ctxs, 3, False, limit=40)
    dec = BeamDecoder(m, beams=3, max_batch=2, sync_every=4, reserve=16)
    assert dec.generate([c.cuda() for c in ctxs]) == ref
    assert [len(r) for r in ref][2:4] == [3, 1]  # contexts ending at the cap: three tokens, and the first only


@pytest.mark.parametrize("beams,score_dtype", [(1, np.float32), (5, np.float32), (16, np.float32), (3, np.float64)])
def test_beam_step_bookkeeping_vs_oracle(cuda, beams, score_dtype):
    """``beam_prepare`` and ``beam_take_over`` against the oracle's row-by-row restatement, bit for bit: random
    states with finished groups, ended rows and EOS / PAD choices, two spare groups of rows past the launch that must
    stay untouched, vocabularies up to the config's, ptr / hist rows of 1-300 columns."""
    from test_oracle import _beam_state

    rng = np.random.default_rng(40 + beams)
    for trial in range(8):
        groups, vocab, cols = int(rng.integers(1, 9)), int(rng.integers(3, 10289)), int(rng.integers(2, 301))
        spare = groups + 2
        st, best, flat = _beam_state(rng, spare, beams, vocab, cols, score_dtype)
        best, flat = best[:groups].copy(), flat[:groups].copy()
        st["k_step"][:] = rng.integers(0, cols, spare)  # includes k = 0 (gen_pos clamps to 0)
        limit = int(rng.integers(5, 600))
        say(f"beam bookkeeping: groups={groups} beams={beams} vocab={vocab} cols={cols} score={score_dtype.__name__}")
        dev = {k: torch.from_numpy(v.copy()).to(cuda) for k, v in st.items()}
        rows = spare * beams
        outs = [torch.full((rows,), -7, dtype=torch.long, device=cuda) for _ in range(2)] + \
               [torch.full((spare,), -7, dtype=torch.long, device=cuda), torch.full((rows,), -7, dtype=torch.long,
                                                                                  device=cuda)]
        kernels.beam_prepare(groups, beams, dev["ctx"], dev["k_step"], dev["group_done"], dev["ptr"], *outs)
        want_ptr = st["ptr"].copy()
        want = ov.beam_prepare(groups, beams, st["ctx"], st["k_step"], st["group_done"], want_ptr)
        r = groups * beams
        np.testing.assert_array_equal(dev["ptr"].cpu().numpy(), want_ptr, err_msg=f"trial {trial}: prepare ptr")
        for got, w, n in zip(outs, want, (r, r, groups, r)):
            got = got.cpu().numpy()
            np.testing.assert_array_equal(got[:n], w, err_msg=f"trial {trial}: prepare")
            assert (got[n:] == -7).all()
        # after the top-k
        dev["k_step"] = torch.from_numpy(st["k_step"].copy()).clamp(min=1).to(cuda)
        st["k_step"] = np.maximum(st["k_step"], 1)
        kernels.beam_take_over(torch.from_numpy(best).to(cuda), torch.from_numpy(flat).to(cuda), vocab, dev["ptr"],
                               dev["hist"], dev["ended"], dev["score"], dev["count"], dev["tok"], dev["k_step"],
                               dev["group_done"], dev["ctx"], limit, 2, 1)
        ref = {k: v.copy() for k, v in st.items()}
        ref["ptr"] = want_ptr
        ov.beam_take_over(best, flat, vocab, ref["ptr"], ref["hist"], ref["ended"], ref["score"], ref["count"],
                          ref["tok"], ref["k_step"], ref["group_done"], ref["ctx"], limit, 2, 1)
        for key in ("ptr", "hist", "ended", "score", "count", "tok", "k_step", "group_done"):
            np.testing.assert_array_equal(dev[key].cpu().numpy(), ref[key], err_msg=f"trial {trial}: {key}")

"""The verify attention's entry point that allocates nothing (``omni_verify_attention_static``), through the C ABI,
against the entry point that takes the caller's workspace and tickets (``omni_verify_attention``): the same kernels
with the same split, so the outputs must be equal bit for bit.  Calls in a row with shrinking shapes share the one
static scratch of the GPU (its partials and tickets keep the previous call's contents), and a captured graph of the
static call replays equal to the eager call."""

import sys

import numpy as np
import pytest
import torch

from omniasr_trt_amd import _lib, kernels

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def case(cuda, rows, t, heads, d, cap, lo, hi, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(rows * t, heads, d, generator=g).to(torch.bfloat16).to(cuda)
    kc = torch.randn(rows, heads, cap, d, generator=g).to(torch.bfloat16).to(cuda)
    vc = torch.randn(rows, heads, cap, d, generator=g).to(torch.bfloat16).to(cuda)
    lengths = torch.randint(lo, hi + 1, (rows,), generator=g).to(cuda)
    keys = -(-(int(lengths.max()) + t) // 256) * 256
    assert keys <= cap
    return q, kc, vc, lengths, keys


# (rows, tokens, heads, head_dim, cache, lengths lo..hi, separate merge launch): the halves kernel (8 x 32 x 128), then
# smaller shapes on split-K with the merge in the last split (tickets) or a merge launch, the wide-head kernel, and the
# halves kernel again on fewer rows.
CALLS = [
    (8, 5, 32, 128, 2560, 750, 2400, True),
    (4, 3, 8, 128, 768, 0, 600, False),
    (8, 5, 8, 512, 1280, 300, 1000, True),
    (2, 1, 4, 128, 512, 1, 300, False),
    (8, 2, 16, 128, 1024, 100, 700, True),
]


def test_static_scratch_equals_caller_workspace(cuda):
    for i, (rows, t, heads, d, cap, lo, hi, separate) in enumerate(CALLS):
        q, kc, vc, lengths, keys = case(cuda, rows, t, heads, d, cap, lo, hi, 100 + i)
        say(f"static scratch call {i}: rows={rows} T={t} heads={heads} d={d} keys={keys} separate={separate}")
        want = kernels.draft_attention(q, kc, vc, lengths, t, keys, d ** -0.5, separate=separate)
        out = torch.full_like(q, float("nan"))
        kernels.verify_attention_static(q, kc, vc, lengths, t, keys, d ** -0.5, out, separate=separate)
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
        # the same call again: the scratch now holds this call's partials and tickets
        kernels.verify_attention_static(q, kc, vc, lengths, t, keys, d ** -0.5, out, separate=separate)
        torch.cuda.synchronize()
        assert torch.equal(out, want), i


def test_raw_c_abi_call(cuda):
    """The entry point called with ctypes and raw pointers, as an FFI caller would."""
    lib = _lib.load()
    q, kc, vc, lengths, keys = case(cuda, 8, 5, 32, 128, 2560, 750, 2400, 7)
    want = kernels.draft_attention(q, kc, vc, lengths, 5, keys, 128 ** -0.5)
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream().cuda_stream
    st = lib.omni_verify_attention_static(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1),
                                          kc.stride(2), kc.size(2), lengths.data_ptr(), 8, 5, 32, 128, keys, 0,
                                          128 ** -0.5, out.data_ptr(), _lib.ATTN_SEPARATE_COMBINE, _lib.BF16, stream)
    assert st == 0
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    # a second, smaller call straight after
    q2, kc2, vc2, len2, keys2 = case(cuda, 3, 4, 16, 128, 512, 10, 400, 8)
    want2 = kernels.draft_attention(q2, kc2, vc2, len2, 4, keys2, 128 ** -0.5, separate=False)
    out2 = torch.empty_like(q2)
    st = lib.omni_verify_attention_static(q2.data_ptr(), kc2.data_ptr(), vc2.data_ptr(), kc2.stride(0),
                                          kc2.stride(1), kc2.stride(2), kc2.size(2), len2.data_ptr(), 3, 4, 16, 128,
                                          keys2, 0, 128 ** -0.5, out2.data_ptr(), 0, _lib.BF16, stream)
    assert st == 0
    torch.cuda.synchronize()
    assert torch.equal(out2, want2)


def test_shapes_beyond_the_scratch_are_refused(cuda):
    """A workspace above the static maximum is an error before any launch; the output is left untouched."""
    q, kc, vc, lengths, _ = case(cuda, 8, 16, 32, 128, 8192, 100, 200, 9)
    need = _lib.load().omni_verify_attention_workspace(8, 16, 32, 128, 8192, 64)
    assert need > _lib.STATIC_WORKSPACE_BYTES
    out = torch.zeros_like(q)
    with pytest.raises(_lib.KernelError, match="workspace"):
        kernels.verify_attention_static(q, kc, vc, lengths, 16, 8192, 128 ** -0.5, out, chunk=64)
    torch.cuda.synchronize()
    assert int(out.abs().sum()) == 0


def test_graph_replays_of_the_static_call(cuda):
    """Captured once (the ticket clear is a fill kernel, so it replays), replayed with new lengths written in place,
    eager calls of both entry points in between; every replay equals the eager call."""
    q, kc, vc, lengths, keys = case(cuda, 8, 5, 32, 128, 2560, 750, 2400, 11)
    out = torch.empty_like(q)
    kernels.verify_attention_static(q, kc, vc, lengths, 5, keys, 128 ** -0.5, out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        graph.capture_begin()
        kernels.verify_attention_static(q, kc, vc, lengths, 5, keys, 128 ** -0.5, out)
        graph.capture_end()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.Generator(device=cuda).manual_seed(12)
    for rep in range(4):
        lengths.copy_(torch.randint(0, keys - 5, lengths.shape, device=cuda, generator=g))
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = kernels.draft_attention(q, kc, vc, lengths, 5, keys, 128 ** -0.5)
        other = torch.empty_like(q[:8])
        kernels.verify_attention_static(q[:8], kc, vc, lengths, 1, keys, 128 ** -0.5, other)  # eager, in between
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep
    assert np.isfinite(out.float().cpu().numpy()).all()


FIRST_CALL_UNDER_CAPTURE = r"""
import sys
sys.path.insert(0, sys.argv[1])
import importlib
import torch
importlib.import_module("omniasr-trt_amd")
from omniasr_trt_amd import _lib
lib = _lib.load()
q = torch.zeros(5, 8, 128, dtype=torch.bfloat16, device="cuda")
kc = torch.zeros(1, 8, 256, 128, dtype=torch.bfloat16, device="cuda")
lengths = torch.tensor([100], device="cuda")
out = torch.zeros_like(q)
def call(stream):
    return lib.omni_verify_attention_static(q.data_ptr(), kc.data_ptr(), kc.data_ptr(), kc.stride(0), kc.stride(1),
                                            kc.stride(2), 256, lengths.data_ptr(), 1, 5, 8, 128, 256, 0, 0.1,
                                            out.data_ptr(), _lib.ATTN_SEPARATE_COMBINE, _lib.BF16, stream)
side = torch.cuda.Stream()
side.wait_stream(torch.cuda.current_stream())
graph = torch.cuda.CUDAGraph()
with torch.cuda.stream(side):
    graph.capture_begin()
    under = call(side.cuda_stream)  # no address yet, stream capturing: refused, nothing recorded
    graph.capture_end()
torch.cuda.synchronize()
init = lib.omni_verify_attention_static_init()
again = lib.omni_verify_attention_static_init()
eager = call(torch.cuda.current_stream().cuda_stream)
torch.cuda.synchronize()
print("statuses", under, init, again, eager, flush=True)
assert under == -1 and init == 0 and again == 0 and eager == 0
"""


def test_first_call_under_capture_is_refused(cuda):
    """In a fresh process, the entry point's first call on the device made under graph capture returns
    OMNI_ERR_INVALID before any lookup or launch (the static scratch has no address yet); after
    ``omni_verify_attention_static_init`` the same call runs."""
    import subprocess
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    say("fresh process: the static entry point's first call under capture")
    res = subprocess.run([sys.executable, "-c", FIRST_CALL_UNDER_CAPTURE, str(root)], capture_output=True, text=True,
                         timeout=300)
    say(res.stdout.strip()[-500:], res.stderr.strip()[-1500:])
    assert res.returncode == 0
    assert "statuses -1 0 0 0" in res.stdout

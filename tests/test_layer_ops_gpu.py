"""The decoder layers' element-wise ops on an MI355X through the C ABI, against torch fp32 / fp64 references of the
same ops: ``rms_norm`` (one rounding after both products, as torch's fused kernel) and ``silu_mul`` (silu rounded to
bf16, then the product: torch's two kernels' rounding, bit for bit)."""

import sys

import pytest
import torch
import torch.nn.functional as F

from omniasr_trt_amd import kernels

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True, file=sys.stderr)


@pytest.mark.parametrize("rows,dim", [(40, 4096), (1, 4096), (8, 4096), (333, 1024), (16384, 4096), (3, 8192), (5, 16)])
def test_rms_norm_vs_fp64_and_torch(cuda, rows, dim):
    say(f"rms_norm rows={rows} dim={dim}")
    g = torch.Generator().manual_seed(rows * 7 + dim)
    x = (torch.randn(rows, dim, generator=g) * 3).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(dim, generator=g)).to(torch.bfloat16)
    got = kernels.rms_norm(x.to(cuda), w.to(cuda), 1e-5).cpu()
    exact = x.double() * torch.rsqrt(x.double().pow(2).mean(-1, keepdim=True) + 1e-5) * w.double()
    # One bf16 rounding of a value computed in fp32: within 2^-8 relative (plus fp32 noise near zero).
    err = (got.double() - exact).abs()
    assert bool((err <= exact.abs() * 2.0 ** -8 + 1e-6).all()), float((err / exact.abs().clamp_min(1e-6)).max())
    # torch's own kernel rounds once too; only the sum of squares' order differs (a last-bit change of rsqrt).
    same = float((got == F.rms_norm(x.to(cuda), (dim,), w.to(cuda), 1e-5).cpu()).float().mean())
    say(f"  identical to F.rms_norm: {same:.6f}")
    assert same >= 0.999


def test_rms_norm_row_stride_and_zero_rows(cuda):
    g = torch.Generator().manual_seed(11)
    big = torch.randn(6, 4096 + 64, generator=g).to(torch.bfloat16).to(cuda)
    x = big[:, :4096]  # rows 4160 elements apart
    w = torch.ones(4096, dtype=torch.bfloat16, device=cuda)
    got = kernels.rms_norm(x, w, 1e-6)
    want = kernels.rms_norm(x.contiguous(), w, 1e-6)
    assert torch.equal(got, want)
    assert kernels.rms_norm(x[:0], w, 1e-6).shape == (0, 4096)
    zero = kernels.rms_norm(torch.zeros(2, 4096, dtype=torch.bfloat16, device=cuda), w, 1e-5)
    assert bool((zero == 0).all())  # 0 * rsqrt(eps): no NaN


@pytest.mark.parametrize("rows,ffn", [(40, 11008), (1, 11008), (8, 8), (1000, 2048), (16384, 11008)])
def test_silu_mul_bit_for_bit_with_torch(cuda, rows, ffn):
    say(f"silu_mul rows={rows} ffn={ffn}")
    g = torch.Generator().manual_seed(rows + ffn)
    gi = (torch.randn(rows, 2 * ffn, generator=g) * 4).to(torch.bfloat16).to(cuda)
    gi[0, :8] = torch.tensor([0.0, -0.0, 88.0, -88.0, 100.0, -100.0, 1e30, -1e30])  # exp overflows both ways
    got = kernels.silu_mul(gi)
    gate, inner = gi.chunk(2, -1)
    want = inner * F.silu(gate)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    exact = inner.double() * (gate.double() * torch.sigmoid(gate.double()))
    fin = torch.isfinite(exact)
    assert bool(((got.double() - exact).abs()[fin] <= exact.abs()[fin] * 2.0 ** -7 + 1e-30).all())


def test_layer_ops_refuse_other_dtypes_and_shapes(cuda):
    x = torch.zeros(4, 4096, device=cuda)
    with pytest.raises(ValueError):
        kernels.rms_norm(x, torch.ones(4096, device=cuda), 1e-5)  # fp32
    with pytest.raises(ValueError):
        kernels.silu_mul(torch.zeros(4, 20, dtype=torch.bfloat16, device=cuda))  # F = 10, not a multiple of 8

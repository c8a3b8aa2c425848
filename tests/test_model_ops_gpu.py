"""The fused residual-add + RMSNorm and SiLU x up kernels (csrc/model_ops.hip, through the C ABI)
against the reference's own torch op chains on the same GPU tensors (model.py:49-55,112-120,
128-138).  The residual add is exact; the normalised rows and the activation keep the reference's
rounding points, so they may differ only where the mean's summation order or the rsqrt / exp
implementation moves an fp32 value across a 16-bit rounding boundary, on a small fraction of
elements: one unit in the last place at that rounding point, which the following multiply by the
weight (about 1) and its own rounding can carry to at most two units in the output."""
import pytest
import torch
import torch.nn.functional as F

from conftest import announce
from kernels.model_ops import add_rmsnorm, silu_mul

pytestmark = pytest.mark.gpu


def torch_rmsnorm(x, w, eps):
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return w * xf.to(x.dtype)


def ulps(a, b):
    """Distance in units in the last place between two 16-bit tensors of one sign pattern."""
    ia = a.view(torch.int16).int()
    ib = b.view(torch.int16).int()
    return torch.where(a.float() == b.float(), 0, (ia - ib).abs())   # +0 == -0


def close_in_ulps(got, want, frac=0.01, max_ulps=2):
    d = ulps(got, want)
    assert d.max().item() <= max_ulps, d.max().item()
    assert (d > 0).float().mean().item() <= frac


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("rows,hidden", [(1, 1536), (16, 1536), (300, 1536), (5, 8), (3, 8192),
                                         (7, 8960 // 2)])
def test_add_rmsnorm_matches_the_torch_chain(dtype, rows, hidden):
    g = torch.Generator().manual_seed(rows * 7 + hidden)
    x = torch.randn(rows, hidden, generator=g).to(dtype).cuda()
    y = (torch.randn(rows, hidden, generator=g) * 0.5).to(dtype).cuda()
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(dtype).cuda()
    announce(f"[gpu] add_rmsnorm {rows}x{hidden} {dtype}")
    r, out = add_rmsnorm(x, w, 1e-6, y=y)
    torch.cuda.synchronize()
    want_r = x + y
    assert torch.equal(r, want_r)
    close_in_ulps(out, torch_rmsnorm(want_r, w, 1e-6))
    # no residual: plain RMSNorm; strided rows; in place residual
    _, out2 = add_rmsnorm(x, w, 1e-6)
    close_in_ulps(out2, torch_rmsnorm(x, w, 1e-6))
    xs = torch.randn(rows, hidden + 64, generator=g).to(dtype).cuda()[:, :hidden]
    _, out3 = add_rmsnorm(xs, w, 1e-6)
    close_in_ulps(out3, torch_rmsnorm(xs, w, 1e-6))
    xi = x.clone()
    r4, out4 = add_rmsnorm(xi, w, 1e-6, y=y, residual_out=xi)
    torch.cuda.synchronize()
    assert r4.data_ptr() == xi.data_ptr() and torch.equal(xi, want_r) and torch.equal(out4, out)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("rows,inter", [(1, 8960), (16, 8960), (257, 8), (40, 1000)])
def test_silu_mul_matches_the_torch_chain(dtype, rows, inter):
    g = torch.Generator().manual_seed(rows + inter)
    gu = (torch.randn(rows, 2 * inter, generator=g) * 3).to(dtype).cuda()
    announce(f"[gpu] silu_mul {rows}x{inter} {dtype}")
    got = silu_mul(gu)
    gate, up = gu.split(inter, dim=-1)
    close_in_ulps(got, F.silu(gate) * up, max_ulps=1)


def test_special_values_pass_through_like_torch():
    x = torch.tensor([[0.0] * 8, [1e4] * 8], dtype=torch.bfloat16).cuda()
    w = torch.ones(8, dtype=torch.bfloat16).cuda()
    _, out = add_rmsnorm(x, w, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(out, torch_rmsnorm(x, w, 1e-6))       # zeros stay zeros (rsqrt(eps))
    gu = torch.tensor([[-100.0, 0.0, 100.0, 5.0, 1.0, 1.0, 1.0, 1.0] + [2.0] * 8],
                      dtype=torch.bfloat16).cuda()
    got = silu_mul(gu)
    close_in_ulps(got, F.silu(gu[:, :8]) * gu[:, 8:], frac=0.2)

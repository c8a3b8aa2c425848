"""mi_fa2_combine: merging partials computed over disjoint key ranges gives the attention over all
the keys.

The partials are built on the CPU by the oracle itself (oracle.sdpa.attention_ref and lse_ref over
key sub-ranges, kernels/test_fa2.py:28-35 and the L of kernels/fa2.py:155-158), so the merge is
checked against the unsplit oracle and nothing else: fp32 outputs and the merged LSE to 1e-5, bf16
outputs to the attention tolerance.  Sub-ranges may be empty (LSE -inf), a row may have none that
saw a key (output 0, LSE -inf), and partial slots past a row's count hold NaN that must not be read.
"""
import pytest
import torch

from conftest import announce
from oracle import sdpa

pytestmark = pytest.mark.gpu


def build(seed, B=7, Hq=12, Hkv=2, T=2, max_parts=4):
    g = torch.Generator().manual_seed(seed)
    lens = [0, 1, 37, 300, 1025, 4096, 129][:B]
    S = max(lens)
    q = torch.randn(B, Hq, T, 128, generator=g)
    k = torch.randn(B, Hkv, S, 128, generator=g)
    v = torch.randn(B, Hkv, S, 128, generator=g)
    part_o = torch.full((max_parts, B, T, Hq, 128), float("nan"))
    part_l = torch.full((max_parts, B, T, Hq), float("nan"))
    counts = []
    for b, n in enumerate(lens):
        P = int(torch.randint(1, max_parts + 1, (1,), generator=g))
        cuts = sorted(torch.randint(0, n + 1, (P - 1,), generator=g).tolist())
        bounds = [0] + cuts + [n]
        for i in range(P):
            lo, hi = bounds[i], bounds[i + 1]
            kb, vb = k[b:b + 1, :, lo:hi], v[b:b + 1, :, lo:hi]
            o = sdpa.attention_ref(q[b:b + 1], kb, vb, False)[0]        # [Hq, T, d]
            lse = sdpa.lse_ref(q[b:b + 1], kb, False)[0]                # [Hq, T]
            part_o[i, b] = o.transpose(0, 1)
            part_l[i, b] = lse.transpose(0, 1)
        counts.append(P)
    want = sdpa.attention_ref(q, k, v, False, lens).permute(0, 2, 1, 3)  # [B, T, Hq, d]
    want_l = sdpa.lse_ref(q, k, False, lens).permute(0, 2, 1)            # [B, T, Hq]
    R = B * T
    n_parts = torch.tensor(counts, dtype=torch.int32).repeat_interleave(T)
    return (part_o.reshape(max_parts, R, Hq, 128), part_l.reshape(max_parts, R, Hq), n_parts,
            want.reshape(R, Hq, 128), want_l.reshape(R, Hq))


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_merge_of_oracle_partials_equals_the_unsplit_oracle(seed):
    from kernels.fa2 import fa2_combine
    po, pl, n_parts, want, want_l = build(seed)
    announce(f"[gpu] combine: oracle partials, seed {seed}")
    o, lse = fa2_combine(po.cuda(), pl.cuda(), n_parts.cuda(), torch.float32, return_lse=True)
    ob = fa2_combine(po.cuda(), pl.cuda(), n_parts.cuda(), torch.bfloat16)
    torch.cuda.synchronize()
    o, lse, ob = o.cpu(), lse.cpu(), ob.float().cpu()
    assert torch.isfinite(o).all()
    assert (o - want).abs().max().item() < 1e-5
    err = (ob - want).abs()
    assert err.max().item() < 1e-2 and err.mean().item() < 1e-3
    # rows of the empty first sequence: zeros and -inf
    assert (o[:2] == 0).all() and torch.isinf(lse[:2]).all() and (lse[:2] < 0).all()
    fin = torch.isfinite(want_l)
    assert torch.equal(fin, torch.isfinite(lse))
    assert (lse[fin] - want_l[fin]).abs().max().item() < 1e-5


def test_merge_without_counts_uses_every_partial_and_strided_outputs():
    from kernels import _lib
    from kernels.fa2 import fa2_combine
    po, pl, n_parts, want, want_l = build(3, max_parts=3)
    # give every row all 3 slots: unused slots become empty ranges (LSE -inf, O NaN: not read)
    for r, n in enumerate(n_parts.tolist()):
        pl[n:, r] = float("-inf")
    announce("[gpu] combine: n_parts NULL, fp16 out into a strided view")
    o = fa2_combine(po.cuda(), pl.cuda(), None, torch.float16)
    torch.cuda.synchronize()
    err = (o.float().cpu() - want).abs()
    assert err.max().item() < 1e-2 and err.mean().item() < 1e-3
    # a strided fp32 output (every other head of a wider buffer) through the C ABI; the heads
    # between stay untouched, and with no partials at all every (row, head) gets zeros
    R, H = want.shape[:2]
    big = torch.full((R, 2 * H, 128), 7.0, dtype=torch.float32, device="cuda")
    view = big[:, 1::2]
    pod, pld = po.cuda(), pl.cuda()
    lib = _lib.load()
    with torch.cuda.device(0):
        _lib.check(lib.mi_fa2_combine(
            2, pod.data_ptr(), pld.data_ptr(), None, R, H, pod.shape[0], 128, _lib.strides(pod, 3),
            _lib.strides(pld, 3), view.data_ptr(), _lib.strides(view, 2), None, None,
            _lib.stream_of(view)))
    torch.cuda.synchronize()
    assert (big[:, 0::2] == 7.0).all()
    assert (view.cpu() - want).abs().max().item() < 1e-5
    with torch.cuda.device(0):
        _lib.check(lib.mi_fa2_combine(
            2, None, None, None, R, H, 0, 128, None, None, view.data_ptr(), _lib.strides(view, 2),
            None, None, _lib.stream_of(view)))
    torch.cuda.synchronize()
    assert (view == 0).all() and (big[:, 0::2] == 7.0).all()


def test_misaligned_contiguous_partials_are_copied_not_refused():
    # a contiguous view that starts 4 bytes into its buffer: the wrapper copies it to an aligned
    # allocation for the kernel's 8-byte loads instead of passing it on (and being refused)
    from kernels.fa2 import fa2_combine
    po, pl, n_parts, want, want_l = build(4, max_parts=2)
    flat = torch.empty(po.numel() + 1, dtype=torch.float32, device="cuda")
    view = flat[1:].view(po.shape)
    view.copy_(po.cuda())
    assert view.is_contiguous() and view.data_ptr() % 8 == 4
    announce("[gpu] combine: contiguous partials at a 4-byte offset")
    o = fa2_combine(view, pl.cuda(), n_parts.cuda(), torch.float32)
    torch.cuda.synchronize()
    assert (o.cpu() - want).abs().max().item() < 1e-5

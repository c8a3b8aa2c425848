"""GPU parity of the general kernel (csrc/fa2_general.hip) against the CPU oracle, through
FlashAttention2Function.apply and the C ABI: the launcher's envelope beyond the engine's shape
(kernels/fa2.py:164-214), i.e. power-of-two head dims 16..256 with d_v free of d (kernels/fa2.py:185)
and fp32 inputs with fp32 dots (kernels/fa2.py:129,147).

Tolerances, against the fp32 oracle:
  * bf16 / fp16 outputs: mean-abs < 1e-3, and every element within 1e-2 plus the rounding of the
    output to its own type (half an ulp: 2^-8 |ref| for bf16, 2^-11 |ref| for fp16).  The second
    term matters only for large outputs: a query that sees 1-3 keys gets an output near a single
    V value, which for N(0,1) data can exceed 4, where half a bf16 ulp alone is 1.6e-2.  (The
    reference's own test allows max-abs 2e-2 flat, kernels/test_fa2.py:25.)
  * fp32 outputs: max-abs < 1e-4 and mean-abs < 1e-5.  Both sides compute in fp32 and differ in
    summation order and in the exponential (v_exp_f32, about 1 ulp), which over at most a few
    thousand keys stays orders of magnitude below this bar.
"""
import math

import pytest
import torch

from conftest import announce
from kernels.fa2 import FlashAttention2Function, fa2_forward
from oracle import sdpa
import workloads as wl

pytestmark = pytest.mark.gpu

DEV = "cuda"
PAD_VALUE = 100.0  # kernels/test_fa2.py:24
BARS = {torch.bfloat16: (1e-2, 1e-3), torch.float16: (1e-2, 1e-3), torch.float32: (1e-4, 1e-5)}
HALF_ULP = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 0.0}
DTYPES = [torch.bfloat16, torch.float16, torch.float32]
IDS = ["bf16", "fp16", "fp32"]


def check_close(out, ref, dtype, what=""):
    max_abs, mean_abs = BARS[dtype]
    out = out.float().cpu()
    assert out.shape == ref.shape, (out.shape, ref.shape)
    assert torch.isfinite(out).all(), f"{what}: non-finite output"
    ref = ref.float()
    err = (out - ref).abs()
    excess = err - (max_abs + HALF_ULP[dtype] * ref.abs())
    assert excess.max().item() < 0, (
        f"{what}: max-abs {err.max().item():.3e} (|ref| there {ref.abs().flatten()[err.argmax()]:.3f})")
    assert err.mean().item() < mean_abs, f"{what}: mean-abs {err.mean().item():.3e}"


def rand(shape, g, dtype):
    return torch.randn(*shape, generator=g).to(dtype)


CASES = [  # kernels/test_fa2.py:17-23
    ("prefill", 300, [300, 300], True),
    ("decode", 1, [1000, 1000], False),
    ("chunked", 64, [500, 500], True),
    ("ragged decode", 1, [1000, 37, 512, 1], False),
    ("ragged prefill", 16, [16, 300, 100], True),
]


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("case", CASES, ids=[c[0].replace(" ", "_") for c in CASES])
def test_reference_cases_at_head_dim_64(case, dtype):
    name, T, lens, causal = case
    B, S = len(lens), max(lens)
    g = torch.Generator().manual_seed(0)
    q = rand((B, 12, T, 64), g, dtype)
    k = rand((B, 2, S, 64), g, dtype)
    v = rand((B, 2, S, 64), g, dtype)
    for b, n in enumerate(lens):
        k[b, :, n:] = PAD_VALUE
        v[b, :, n:] = PAD_VALUE
    announce(f"[gpu] general: reference case {name} d=64 {dtype}")
    out = FlashAttention2Function.apply(q.to(DEV), k.to(DEV), v.to(DEV), causal,
                                        torch.tensor(lens, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    check_close(out, sdpa.attention_ref(q, k, v, causal, lens), dtype, name)


# (d, d_v): every head dim at least once on each side, equal and unequal pairs
DIMS = [(16, 16), (32, 64), (64, 32), (256, 256), (256, 16), (16, 256), (128, 64), (128, 128)]


@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
@pytest.mark.parametrize("dims", DIMS, ids=[f"d{a}_dv{b}" for a, b in DIMS])
@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_head_dims_and_dtypes(dtype, dims, causal):
    d, d_v = dims
    g = torch.Generator().manual_seed(d * 7 + d_v)
    B, Hq, Hkv, T, S, lens = 2, 6, 2, 37, 70, [70, 23]
    q = rand((B, Hq, T, d), g, dtype)
    k = rand((B, Hkv, S, d), g, dtype)
    v = rand((B, Hkv, S, d_v), g, dtype)
    announce(f"[gpu] general: d={d} d_v={d_v} {dtype} causal={causal}")
    out, lse = fa2_forward(q.to(DEV), k.to(DEV), v.to(DEV), causal,
                           torch.tensor(lens, dtype=torch.int32, device=DEV), return_lse=True)
    torch.cuda.synchronize()
    check_close(out, sdpa.attention_ref(q, k, v, causal, lens), dtype, f"d={d} d_v={d_v}")
    want = sdpa.lse_ref(q, k, causal, lens)
    fin = torch.isfinite(want)
    assert torch.equal(fin, torch.isfinite(lse.cpu()))  # row 1's first queries see no key
    # 16-bit: the row sum adds P as rounded for the PV product (unit roundoff 2^-8 for bf16), so
    # |dLSE| <= log(1 + 2^-8) = 3.9e-3 plus the scores' own error; fp32: no rounding.
    bar = 1e-4 if dtype == torch.float32 else math.log1p(2.0 ** -8) + 1e-3
    assert (lse.cpu()[fin] - want[fin]).abs().max().item() < bar


def test_plumbing_workload_in_fp32():
    # 1 x 12q/2kv x 512 x 128, fp32 N(0,1), causal: the workload the reference runs through its
    # fp32 SDPA fallback (model.py:104-107), here in fp32 on the GPU.
    q, k, v = wl.prefill_single(512, dtype=torch.float32, seed=0)
    announce("[gpu] general: fp32 1x12x512 causal")
    out = FlashAttention2Function.apply(q.to(DEV), k.to(DEV), v.to(DEV), True, None)
    torch.cuda.synchronize()
    check_close(out, sdpa.attention_ref(q, k, v, True), torch.float32, "plumbing fp32")


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_padding_is_never_read(dtype):
    # NaN and inf past each row's kv_len: a load of them would poison the output.
    g = torch.Generator().manual_seed(5)
    lens = [40, 7, 0]
    q = rand((3, 4, 9, 32), g, dtype)
    k = rand((3, 2, 48, 32), g, dtype)
    v = rand((3, 2, 48, 64), g, dtype)
    for b, n in enumerate(lens):
        k[b, :, n:] = float("nan")
        v[b, :, n:] = float("inf")
    announce(f"[gpu] general: NaN/inf padding {dtype}")
    for causal in (True, False):
        out, lse = fa2_forward(q.to(DEV), k.to(DEV), v.to(DEV), causal,
                               torch.tensor(lens, dtype=torch.int32, device=DEV), return_lse=True)
        torch.cuda.synchronize()
        kc, vc = k.clone(), v.clone()
        for b, n in enumerate(lens):
            kc[b, :, n:] = 0
            vc[b, :, n:] = 0
        check_close(out, sdpa.attention_ref(q, kc, vc, causal, lens), dtype, f"causal={causal}")
        assert torch.equal(out[2].cpu().float(), torch.zeros(4, 9, 64))  # the empty row
        assert torch.isinf(lse[2]).all() and (lse[2] < 0).all()


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_strided_views(dtype):
    # [B, T, H, d] activations viewed as [B, H, T, d], as model.py hands them over.
    g = torch.Generator().manual_seed(6)
    B, T, S = 2, 50, 50
    q = rand((B, T, 8, 64), g, dtype).to(DEV).transpose(1, 2)
    k = rand((B, S, 4, 64), g, dtype).to(DEV).transpose(1, 2)
    v = rand((B, S, 4, 32), g, dtype).to(DEV).transpose(1, 2)
    announce(f"[gpu] general: strided views {dtype}")
    out = FlashAttention2Function.apply(q, k, v, True, None)
    torch.cuda.synchronize()
    ref = sdpa.attention_ref(q.cpu(), k.cpu(), v.cpu(), True)
    check_close(out, ref, dtype, "strided")
    assert out.is_contiguous() and out.shape == (B, 8, T, 32)


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_long_rows_and_single_queries(dtype):
    # decode-shaped (T = 1) rows of up to 3000 keys, and T > 64 (several work-groups per head)
    g = torch.Generator().manual_seed(7)
    lens = [3000, 1, 1777]
    q = rand((3, 12, 1, 256), g, dtype)
    k = rand((3, 2, 3000, 256), g, dtype)
    v = rand((3, 2, 3000, 128), g, dtype)
    announce(f"[gpu] general: decode d=256 d_v=128 {dtype}")
    out = FlashAttention2Function.apply(q.to(DEV), k.to(DEV), v.to(DEV), False,
                                        torch.tensor(lens, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    check_close(out, sdpa.attention_ref(q, k, v, False, lens), dtype, "decode")
    q2 = rand((1, 4, 200, 64), g, dtype)
    k2 = rand((1, 1, 1000, 64), g, dtype)
    v2 = rand((1, 1, 1000, 64), g, dtype)
    announce(f"[gpu] general: 200 queries over 1000 keys {dtype}")
    out = FlashAttention2Function.apply(q2.to(DEV), k2.to(DEV), v2.to(DEV), True, None)
    torch.cuda.synchronize()
    check_close(out, sdpa.attention_ref(q2, k2, v2, True), dtype, "chunked MQA")


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
def test_both_work_splits(dtype, causal):
    """The launcher picks the LDS-staged kernel (64 query rows per work-group, K/V shared by its 4
    waves) when there are at least 64 query rows and 256 such work-groups, else the key-split one
    (16 rows per work-group, keys split over its 4 waves): shapes on both sides of that line."""
    g = torch.Generator().manual_seed(9)
    for B, Hq, Hkv, T, S, d, d_v in ((4, 16, 4, 256, 300, 64, 64),     # 4*16*4 = 256: LDS-staged
                                     (4, 16, 4, 256, 300, 32, 128),
                                     (4, 15, 5, 256, 300, 64, 64),      # 4*15*4 = 240: key-split
                                     (2, 8, 2, 63, 500, 128, 32)):      # 63 rows: key-split
        if dtype != torch.float32 and d == d_v == 128:
            continue
        q = rand((B, Hq, T, d), g, dtype)
        k = rand((B, Hkv, S, d), g, dtype)
        v = rand((B, Hkv, S, d_v), g, dtype)
        lens = [S, S - 37, T, 200][:B]
        announce(f"[gpu] general: B={B} Hq={Hq} T={T} S={S} d={d} d_v={d_v} {dtype} causal={causal}")
        out, lse = fa2_forward(q.to(DEV), k.to(DEV), v.to(DEV), causal,
                               torch.tensor(lens, dtype=torch.int32, device=DEV), return_lse=True)
        torch.cuda.synchronize()
        check_close(out, sdpa.attention_ref(q, k, v, causal, lens), dtype, f"B={B} Hq={Hq} T={T}")
        want = sdpa.lse_ref(q, k, causal, lens)
        fin = torch.isfinite(want)
        assert torch.equal(fin, torch.isfinite(lse.cpu()))
        bar = 1e-4 if dtype == torch.float32 else math.log1p(2.0 ** -8) + 1e-3
        assert (lse.cpu()[fin] - want[fin]).abs().max().item() < bar


def test_general_kernel_is_deterministic():
    g = torch.Generator().manual_seed(8)
    q = rand((2, 6, 33, 64), g, torch.bfloat16).to(DEV)
    k = rand((2, 3, 90, 64), g, torch.bfloat16).to(DEV)
    v = rand((2, 3, 90, 64), g, torch.bfloat16).to(DEV)
    announce("[gpu] general: repeat calls")
    a = FlashAttention2Function.apply(q, k, v, True, None)
    b = FlashAttention2Function.apply(q, k, v, True, None)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


ALL_DIMS = (16, 32, 64, 128, 256)


@pytest.mark.parametrize("d", ALL_DIMS, ids=[f"d{x}" for x in ALL_DIMS])
@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_staged_kernel_every_head_dim_pair(dtype, d):
    """Every (d, d_v) pair on the LDS-staged general kernel (64 query rows per work-group, K/V
    staged in LDS): B=4, Hq=16, T=256 is 256 such work-groups, which reaches it on MI355X's 256
    CUs.  Covers its 16-bit d=16 path (16x16x16 scores), the 16-bit and fp32 instantiations
    without the register prefetch ((d + d_v) x element size > 512 bytes, e.g. bf16 256/256 and
    fp32 256/256 with about 130 KB of LDS), and d_v = 256; causal and not, ragged rows."""
    from kernels import _lib
    assert 4 * 16 * 4 >= _lib.launch_plan()["num_cus"], "shape must reach the staged kernel"
    B, Hq, Hkv, T, S = 4, 16, 4, 256, 300
    lens = [300, 263, 256, 200]
    for d_v in ALL_DIMS:
        if dtype != torch.float32 and d == d_v == 128:
            continue  # the MFMA prefill kernel's shape, covered by tests/test_fa2_gpu.py
        g = torch.Generator().manual_seed(d * 1000 + d_v)
        q = rand((B, Hq, T, d), g, dtype)
        k = rand((B, Hkv, S, d), g, dtype)
        v = rand((B, Hkv, S, d_v), g, dtype)
        for b, n in enumerate(lens):
            k[b, :, n:] = PAD_VALUE
            v[b, :, n:] = PAD_VALUE
        for causal in (True, False):
            announce(f"[gpu] general staged: d={d} d_v={d_v} {dtype} causal={causal}")
            out, lse = fa2_forward(q.to(DEV), k.to(DEV), v.to(DEV), causal,
                                   torch.tensor(lens, dtype=torch.int32, device=DEV),
                                   return_lse=True)
            torch.cuda.synchronize()
            check_close(out, sdpa.attention_ref(q, k, v, causal, lens), dtype,
                        f"staged d={d} d_v={d_v} causal={causal}")
            want = sdpa.lse_ref(q, k, causal, lens)
            fin = torch.isfinite(want)
            assert torch.equal(fin, torch.isfinite(lse.cpu()))
            bar = 1e-4 if dtype == torch.float32 else math.log1p(2.0 ** -8) + 1e-3
            assert (lse.cpu()[fin] - want[fin]).abs().max().item() < bar

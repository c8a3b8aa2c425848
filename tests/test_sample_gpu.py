"""The fused sampler kernel (csrc/sample.hip, through the C ABI) against the sampler oracle.

Integer results, so the bar is equality: the kernel draws the same token as the float64 oracle on
every row whose two best race scores are further apart than fp32 rounding of the scores can move
them (the kernel forms logit / T - ln(-ln U) in fp32); rows inside that margin are counted and
must be rare.  The distribution is checked separately against softmax(logits / T)."""
import numpy as np
import pytest
import torch
from scipy import stats

from conftest import announce
from kernels.sample import sample_tokens
from oracle import sample as osample

pytestmark = pytest.mark.gpu
DEV = "cuda"


def check_against_oracle(logits, temperature, seed, offset, margin=1e-4):
    got = sample_tokens(logits, temperature, seed, offset).cpu().numpy()
    lg = logits.float().cpu().numpy().astype(np.float64)
    want = osample.sample(lg, temperature, seed, offset)
    s = osample.scores(lg, temperature, seed, offset)
    s = np.where(np.isnan(s), -np.inf, s)
    if s.shape[1] > 1:
        top2 = np.sort(s, axis=1)[:, -2:]
        near = (top2[:, 1] - top2[:, 0]) <= margin * np.maximum(1.0, np.abs(top2[:, 1]))
    else:
        near = np.zeros(s.shape[0], dtype=bool)
    bad = (got != want) & ~near
    assert not bad.any(), (np.nonzero(bad)[0][:8], got[bad][:8], want[bad][:8])
    assert near.mean() < 0.05
    return got


@pytest.mark.parametrize("temperature", [1.0, 0.7])
def test_vocab_151936_bf16_matches_oracle(temperature):
    g = torch.Generator().manual_seed(0)
    logits = (torch.randn(16, 151936, generator=g) * 2).to(torch.bfloat16).to(DEV)
    announce(f"[gpu] sampler 16 x 151936 bf16, T={temperature}")
    for seed, offset in ((0, 0), (1234, 7), (2**63 + 5, 2**32 + 9)):
        check_against_oracle(logits, temperature, seed, offset)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
@pytest.mark.parametrize("vocab", [1, 5, 1001, 8192, 8193, 40000])
def test_dtypes_and_ragged_vocab(dtype, vocab):
    g = torch.Generator().manual_seed(vocab)
    logits = torch.randn(9, vocab, generator=g).to(dtype).to(DEV)
    announce(f"[gpu] sampler 9 x {vocab} {dtype}")
    got = check_against_oracle(logits, 1.0, 42, 3)
    assert ((got >= 0) & (got < vocab)).all()


def test_strided_rows():
    g = torch.Generator().manual_seed(3)
    full = torch.randn(6, 20000, generator=g).to(torch.bfloat16).to(DEV)
    announce("[gpu] sampler strided rows")
    check_against_oracle(full[:, :12345], 0.9, 5, 1)


def test_greedy_is_argmax_with_lowest_index_ties():
    g = torch.Generator().manual_seed(4)
    logits = torch.randn(32, 30000, generator=g).to(DEV)
    logits[0, 100] = logits[0, 20000] = 50.0     # a tie across chunks: index 100 wins
    announce("[gpu] sampler greedy")
    got = sample_tokens(logits, 0.0, 0, 0).cpu()
    want = logits.cpu().argmax(1).to(torch.int32)
    assert torch.equal(got, want) and got[0].item() == 100


def test_special_values():
    logits = torch.zeros(4, 20000)
    logits[0, :] = float("nan")
    logits[0, 17] = 1.0                    # the only candidate among NaNs
    logits[1, :] = float("-inf")           # no candidate
    logits[2, :] = float("nan")            # no candidate
    logits[3, :] = float("-inf")
    logits[3, 12000] = 0.0
    announce("[gpu] sampler NaN / -inf rows")
    for t in (1.0, 0.0):
        got = sample_tokens(logits.to(DEV), t, 9, 0).cpu().tolist()
        assert got == [17, -1, -1, 12000], t


@pytest.mark.parametrize("temperature", [1.0, 0.5])
def test_kernel_draws_follow_the_softmax(temperature):
    lg = torch.tensor([1.0, -0.5, 2.0, 0.0, 0.7, -2.0])
    n = 60000
    announce(f"[gpu] sampler distribution, {n} rows, T={temperature}")
    tokens = sample_tokens(lg.repeat(n, 1).to(DEV), temperature, 77, 0).cpu().numpy()
    x = lg.double().numpy() / temperature
    probs = np.exp(x - x.max()) / np.exp(x - x.max()).sum()
    counts = np.bincount(tokens, minlength=6)
    assert stats.chisquare(counts, probs * n).pvalue > 1e-4


def test_repeat_calls_are_deterministic_and_offsets_differ():
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(64, 50000, generator=g).to(torch.bfloat16).to(DEV)
    announce("[gpu] sampler determinism")
    a = sample_tokens(logits, 1.0, 1, 0)
    assert torch.equal(a, sample_tokens(logits, 1.0, 1, 0))
    assert (a != sample_tokens(logits, 1.0, 1, 1)).float().mean().item() > 0.5

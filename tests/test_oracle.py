"""Pins the CPU oracle before any GPU result is compared with it.

oracle.sdpa.attention_ref (the reference's fp32 SDPA oracle, kernels/test_fa2.py:28-35) is checked
against an independent float64 brute force, against closed forms, and against invariants that a
plausible mistake (top-left instead of bottom-right causal alignment, wrong GQA head mapping, keys
leaking past kv_len, a missing scale) would break.  Each planted mistake is planted in a copy of
the brute force, on the CPU, to show the checks would notice it.
"""
import math

import numpy as np
import pytest
import torch

from oracle import brute, paged, sdpa


def _rand(shape, g, dtype=torch.float32):
    return torch.randn(*shape, generator=g).to(dtype)


# (B, Hq, Hkv, T, S, kv_lens, causal): small versions of the reference's CASES
# (kernels/test_fa2.py:17-23) plus the edge cases the drop-in must handle.
SMALL = [
    (2, 12, 2, 9, 9, [9, 9], True),           # prefill
    (2, 12, 2, 1, 23, [23, 23], False),       # decode
    (2, 12, 2, 4, 11, [11, 11], True),        # chunked: T < S, bottom-right causal
    (4, 12, 2, 1, 17, [17, 5, 9, 1], False),  # ragged decode
    (3, 12, 2, 3, 15, [3, 15, 7], True),      # ragged prefill
    (2, 4, 4, 5, 5, [5, 2], True),            # MHA; row 1 has queries that see no key
    (1, 6, 1, 6, 4, [4], True),               # T > kv_len: first 2 queries see nothing
    (2, 12, 2, 3, 6, [0, 6], True),           # an empty row
]


@pytest.mark.parametrize("case", SMALL, ids=[str(i) for i in range(len(SMALL))])
def test_sdpa_oracle_matches_fp64_brute_force(case):
    B, Hq, Hkv, T, S, lens, causal = case
    g = torch.Generator().manual_seed(1)
    d = 16
    q, k, v = _rand((B, Hq, T, d), g), _rand((B, Hkv, S, d), g), _rand((B, Hkv, S, d), g)
    want, want_lse = brute.attention_f64(q, k, v, causal, lens)
    got = sdpa.attention_ref(q, k, v, causal, lens)
    assert np.abs(got.numpy() - want).max() < 2e-6
    got_lse = sdpa.lse_ref(q, k, causal, lens).numpy()
    fin = np.isfinite(want_lse)
    assert np.array_equal(fin, np.isfinite(got_lse))
    assert np.abs(got_lse[fin] - want_lse[fin]).max() < 2e-5


@pytest.mark.parametrize("d,d_v", [(32, 64), (64, 16), (256, 32)])
def test_sdpa_oracle_matches_fp64_brute_force_when_d_v_differs(d, d_v):
    # The launcher takes V with its own head dim (kernels/fa2.py:172,185); the scale stays
    # 1/sqrt(d) of Q and K (kernels/fa2.py:174).
    g = torch.Generator().manual_seed(4)
    B, Hq, Hkv, T, S, lens = 2, 4, 2, 5, 9, [9, 4]
    q, k, v = _rand((B, Hq, T, d), g), _rand((B, Hkv, S, d), g), _rand((B, Hkv, S, d_v), g)
    for causal in (True, False):
        want, want_lse = brute.attention_f64(q, k, v, causal, lens)
        got = sdpa.attention_ref(q, k, v, causal, lens)
        assert got.shape == (B, Hq, T, d_v)
        assert np.abs(got.numpy() - want).max() < 2e-6
        fin = np.isfinite(want_lse)
        assert np.abs(sdpa.lse_ref(q, k, causal, lens).numpy()[fin] - want_lse[fin]).max() < 2e-5
    # planted mistake: a scale taken from V's head dim moves the output
    bad, _ = brute.attention_f64(q * math.sqrt(d / d_v), k, v, True, lens)
    assert np.abs(bad - brute.attention_f64(q, k, v, True, lens)[0]).max() > 1e-2


def test_brute_force_matches_softmax_formula_at_full_head_dim():
    # d = 128 and GQA 6:1 as in the engine; compares against a vectorised textbook softmax.
    g = torch.Generator().manual_seed(2)
    q, k, v = _rand((1, 12, 5, 128), g), _rand((1, 2, 7, 128), g), _rand((1, 2, 7, 128), g)
    out, _ = brute.attention_f64(q, k, v, True, None)
    qd, kd, vd = (x.double().numpy() for x in (q, k, v))
    kd, vd = np.repeat(kd, 6, axis=1), np.repeat(vd, 6, axis=1)
    s = np.einsum("bhid,bhjd->bhij", qd, kd) / math.sqrt(128)
    i, j = np.arange(5)[:, None], np.arange(7)[None, :]
    s = np.where(j <= i + 2, s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    want = np.einsum("bhij,bhjd->bhid", p / p.sum(-1, keepdims=True), vd)
    assert np.abs(out - want).max() < 1e-12


def test_closed_forms():
    g = torch.Generator().manual_seed(3)
    # one visible key: the output is that key's value, exactly
    q, k, v = _rand((1, 12, 1, 128), g), _rand((1, 2, 1, 128), g), _rand((1, 2, 1, 128), g)
    out = sdpa.attention_ref(q, k, v, False)
    assert torch.equal(out[0, :6, 0], v[0, 0, 0].expand(6, 128))
    assert torch.equal(out[0, 6:, 0], v[0, 1, 0].expand(6, 128))
    # constant V: the output is that constant whatever the weights
    q, k = _rand((2, 12, 4, 128), g), _rand((2, 2, 9, 128), g)
    v = torch.full((2, 2, 9, 128), 0.375)
    out = sdpa.attention_ref(q, k, v, True, [9, 6])
    assert torch.allclose(out, torch.full_like(out, 0.375), atol=1e-6)
    # zero queries: uniform weights, lse = log(number of visible keys), output = mean of values
    q = torch.zeros(1, 12, 3, 128)
    k, v = _rand((1, 2, 8, 128), g), _rand((1, 2, 8, 128), g)
    lse = sdpa.lse_ref(q, k, True, [8])
    assert torch.allclose(lse[0, 0], torch.log(torch.tensor([6.0, 7.0, 8.0])), atol=1e-6)
    out = sdpa.attention_ref(q, k, v, True, [8])
    assert torch.allclose(out[0, 0, 2], v[0, 0].mean(0), atol=1e-6)
    assert torch.allclose(out[0, 0, 0], v[0, 0, :6].mean(0), atol=1e-6)


def test_padding_past_kv_len_never_reaches_the_output():
    # kernels/test_fa2.py:24,47-49: padding filled with 100 would show up as a large error.
    g = torch.Generator().manual_seed(4)
    q, k, v = _rand((2, 12, 3, 128), g), _rand((2, 2, 10, 128), g), _rand((2, 2, 10, 128), g)
    clean = sdpa.attention_ref(q, k, v, True, [10, 6])
    k2, v2 = k.clone(), v.clone()
    k2[1, :, 6:] = 100.0
    v2[1, :, 6:] = float("nan")
    assert torch.equal(sdpa.attention_ref(q, k2, v2, True, [10, 6]), clean)


def _brute_top_left(q, k, v, lens):
    # planted mistake: causal mask aligned top-left (j <= i) instead of bottom-right
    out = np.zeros(q.shape)
    rep = q.shape[1] // k.shape[1]
    for b, n in enumerate(lens):
        for h in range(q.shape[1]):
            for i in range(q.shape[2]):
                hi = min(n, i + 1)
                s = k[b, h // rep, :hi].double().numpy() @ q[b, h, i].double().numpy() / math.sqrt(q.shape[-1])
                w = np.exp(s - s.max())
                out[b, h, i] = w @ v[b, h // rep, :hi].double().numpy() / w.sum()
    return out


def test_planted_mistakes_are_caught():
    g = torch.Generator().manual_seed(5)
    B, Hq, Hkv, T, S = 2, 12, 2, 4, 11
    q, k, v = _rand((B, Hq, T, 16), g), _rand((B, Hkv, S, 16), g), _rand((B, Hkv, S, 16), g)
    ref = sdpa.attention_ref(q, k, v, True, [11, 8]).numpy()
    # top-left causal alignment differs when T < kv_len
    assert np.abs(_brute_top_left(q, k, v, [11, 8]) - ref).max() > 0.1
    # wrong GQA mapping (h % Hkv instead of h // group)
    k_wrong = k[:, [h % Hkv for h in range(Hq)]]
    v_wrong = v[:, [h % Hkv for h in range(Hq)]]
    bad, _ = brute.attention_f64(q, k_wrong, v_wrong, True, [11, 8])
    assert np.abs(bad - ref).max() > 0.1
    # keys past kv_len leaking in
    bad, _ = brute.attention_f64(q, k, v, True, [11, 11])
    assert np.abs(bad[1] - ref[1]).max() > 0.05
    # missing 1/sqrt(d) scale
    bad, _ = brute.attention_f64(q * 4.0, k, v, True, [11, 8])
    assert np.abs(bad - ref).max() > 0.05


def test_varlen_oracle_is_per_row_padded_oracle():
    g = torch.Generator().manual_seed(6)
    lens = [5, 1, 12, 7]
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    q, k, v = _rand((cu[-1], 12, 16), g), _rand((cu[-1], 2, 16), g), _rand((cu[-1], 2, 16), g)
    got = sdpa.varlen_ref(q, k, v, cu, cu, True)
    for b, n in enumerate(lens):
        s, e = cu[b], cu[b + 1]
        want, _ = brute.attention_f64(q[s:e].transpose(0, 1)[None], k[s:e].transpose(0, 1)[None],
                                      v[s:e].transpose(0, 1)[None], True)
        assert np.abs(got[s:e].transpose(0, 1).numpy() - want[0]).max() < 2e-6


def test_paged_gather_restates_dense_layout():
    g = torch.Generator().manual_seed(7)
    bs, lens = 16, [37, 5, 64, 16]
    S = max(lens)
    dense_k = _rand((len(lens), 2, S, 8), g)
    num_blocks = 20
    tables = paged.random_tables(lens, bs, num_blocks, g)
    pool = torch.full((num_blocks * bs, 2, 8), float("nan"))
    paged.scatter_rows(dense_k, lens, tables, pool, bs)
    got = paged.gather_dense(pool, tables, S, bs)
    assert got.shape == dense_k.shape
    for b, n in enumerate(lens):
        assert torch.equal(got[b, :, :n], dense_k[b, :, :n])
    # slot arithmetic of kv_cache.py:15-16
    assert paged.slot_of([7, 3], 17, 16) == 3 * 16 + 1
    # blocks are distinct across rows
    flat = [x for t in tables for x in t]
    assert len(flat) == len(set(flat))

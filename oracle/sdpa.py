"""fp32 SDPA oracle (test infrastructure only; see oracle/__init__.py).

Restates the reference's correctness oracle, kernels/test_fa2.py:28-35 (`reference`) and its use at
kernels/test_fa2.py:54-57 (each row cut to its own kv_len keys), which is also the model's CPU path
(model.py:102-107 with repeat_kv from model.py:70-75).
"""
import math

import torch
import torch.nn.functional as F


def repeat_kv(x, n_rep):
    """[B, Hkv, S, d] -> [B, Hkv*n_rep, S, d]; query head h reads kv head h // n_rep
    (model.py:70-75, kernels/fa2.py:53)."""
    if n_rep == 1:
        return x
    b, h, s, d = x.shape
    return x[:, :, None].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)


def bottom_right_mask(T, S, device=None):
    """[T, S] bool: query i sees key j iff j <= i + (S - T) (kernels/test_fa2.py:31-33,
    kernels/fa2.py:109-111)."""
    return torch.arange(S, device=device)[None, :] <= torch.arange(T, device=device)[:, None] + (S - T)


def _sdpa_row(q, k, v, is_causal):
    # q [1, Hq, T, d], k/v [1, Hkv, n, d] -> fp32 [1, Hq, T, d]
    q = q.float()
    n_rep = q.shape[1] // k.shape[1]
    k = repeat_kv(k.float(), n_rep)
    v = repeat_kv(v.float(), n_rep)
    T, S = q.shape[2], k.shape[2]
    if S == 0:
        return torch.zeros(q.shape[:-1] + (v.shape[-1],), dtype=torch.float32)
    mask = bottom_right_mask(T, S, q.device) if is_causal else None
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask)


def attention_ref(q, k, v, is_causal, kv_lens=None):
    """fp32 attention of a padded batch, each row on its own first kv_lens[b] keys.

    q [B, Hq, T, d], k/v [B, Hkv, S, d] (any float dtype, CPU), kv_lens: list/tensor of B ints or
    None (= S).  A query that sees no key comes out as 0, as fp32 SDPA gives it.
    """
    B, S = q.shape[0], k.shape[2]
    lens = [S] * B if kv_lens is None else [int(x) for x in kv_lens]
    outs = [_sdpa_row(q[b:b + 1], k[b:b + 1, :, :n], v[b:b + 1, :, :n], is_causal)
            for b, n in enumerate(lens)]
    return torch.cat(outs, 0)


def lse_ref(q, k, is_causal, kv_lens=None):
    """fp32 [B, Hq, T] log-sum-exp of scale * q k^T over the keys each query sees
    (-inf where it sees none): the L of kernels/fa2.py:155-158."""
    B, Hq, T, d = q.shape
    S = k.shape[2]
    lens = [S] * B if kv_lens is None else [int(x) for x in kv_lens]
    out = torch.empty(B, Hq, T)
    for b, n in enumerate(lens):
        kk = repeat_kv(k[b:b + 1, :, :n].float(), Hq // k.shape[1])
        s = (q[b:b + 1].float() @ kk.transpose(-1, -2)) / math.sqrt(d)
        if is_causal:
            s = s.masked_fill(~bottom_right_mask(T, n), float("-inf"))
        out[b] = torch.logsumexp(s, dim=-1)[0] if n > 0 else float("-inf")
    return out


def varlen_ref(q, k, v, cu_q, cu_k, is_causal):
    """Packed batch: q [total_q, Hq, d], k/v [total_k, Hkv, d], cu_* lists of B+1 offsets.
    Returns fp32 [total_q, Hq, d]."""
    outs = []
    for b in range(len(cu_q) - 1):
        qs, qe, ks, ke = int(cu_q[b]), int(cu_q[b + 1]), int(cu_k[b]), int(cu_k[b + 1])
        qb = q[qs:qe].transpose(0, 1)[None]
        kb = k[ks:ke].transpose(0, 1)[None]
        vb = v[ks:ke].transpose(0, 1)[None]
        outs.append(_sdpa_row(qb, kb, vb, is_causal)[0].transpose(0, 1))
    return torch.cat(outs, 0)

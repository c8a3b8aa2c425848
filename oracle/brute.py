"""float64 brute-force attention (test infrastructure only; see oracle/__init__.py).

The textbook definition, written out independently of torch's SDPA so that it can pin
oracle.sdpa on small shapes: for every (row b, query head h, query i) take the keys the query sees
(j < kv_len[b] and, if causal, j <= i + kv_len[b] - T: kernels/fa2.py:109-111,132-138), with kv
head h // (Hq/Hkv) (kernels/fa2.py:53), form s_j = q.k_j / sqrt(d), and return
sum_j softmax(s)_j v_j (0 if no key is visible) plus logsumexp(s).
"""
import numpy as np


def attention_f64(q, k, v, is_causal, kv_lens=None):
    """q [B,Hq,T,d], k/v [B,Hkv,S,d] array-likes -> (out [B,Hq,T,d_v], lse [B,Hq,T]) float64."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Hq, T, d = q.shape
    Hkv, S = k.shape[1], k.shape[2]
    rep = Hq // Hkv
    lens = [S] * B if kv_lens is None else [int(x) for x in kv_lens]
    out = np.zeros((B, Hq, T, v.shape[-1]))
    lse = np.full((B, Hq, T), -np.inf)
    scale = 1.0 / np.sqrt(d)
    for b in range(B):
        n = lens[b]
        for h in range(Hq):
            kh, vh = k[b, h // rep], v[b, h // rep]
            for i in range(T):
                hi = min(n, i + n - T + 1) if is_causal else n
                if hi <= 0:
                    continue
                s = (kh[:hi] @ q[b, h, i]) * scale
                m = s.max()
                w = np.exp(s - m)
                out[b, h, i] = (w @ vh[:hi]) / w.sum()
                lse[b, h, i] = m + np.log(w.sum())
    return out, lse

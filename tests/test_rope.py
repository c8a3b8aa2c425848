"""Fused RoPE + paged KV write: the oracle restatement pinned on the CPU, the HIP kernel checked
bitwise against it on the GPU (model.py:58-65,92-96, kv_cache.py:108-115)."""
import math

import pytest
import torch

from conftest import announce
from oracle import rope as orope

N_Q, N_KV, D = 12, 2, 128


# --- oracle pinning (CPU) -------------------------------------------------------------------

def test_position_zero_is_identity():
    x = torch.randn(5, 3, D).to(torch.bfloat16)
    cos, sin = orope.rope_cos_sin(torch.zeros(5, dtype=torch.long))
    assert torch.equal(orope.apply_rope(x, cos[:, None], sin[:, None]), x)


def test_quarter_turn_is_rotate_half():
    x = torch.randn(4, 2, D).to(torch.bfloat16)
    cos, sin = torch.zeros(4, 1, D, dtype=torch.bfloat16), torch.ones(4, 1, D, dtype=torch.bfloat16)
    out = orope.apply_rope(x, cos, sin)
    # rotate_half by hand: first half takes -x[64:], second half takes x[:64]
    want = torch.cat((-x[..., 64:], x[..., :64]), dim=-1)
    assert torch.equal(out, want)


def _tables_f64(pos):
    inv = 1.0 / (1_000_000.0 ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    ang = pos.double()[:, None] * inv[None, :]
    ang = torch.cat((ang, ang), dim=-1)
    return ang.cos(), ang.sin()


def test_rotation_preserves_pair_norms_and_composes():
    x = torch.randn(6, 2, D, dtype=torch.float64)
    pa, pb = torch.tensor([3, 17, 250, 1000, 4095, 70000]), torch.tensor([5, 1, 9, 123, 1, 3])
    ca, sa = _tables_f64(pa)
    cb, sb = _tables_f64(pb)
    cab, sab = _tables_f64(pa + pb)
    ya = orope.apply_rope(x, ca[:, None], sa[:, None])
    norm = lambda t: t[..., :64] ** 2 + t[..., 64:] ** 2
    assert torch.allclose(norm(ya), norm(x), rtol=1e-12, atol=1e-12)
    yab = orope.apply_rope(ya, cb[:, None], sb[:, None])
    assert torch.allclose(yab, orope.apply_rope(x, cab[:, None], sab[:, None]), atol=1e-9)


def test_cos_sin_tables_follow_the_fp32_angles():
    """model.py:151-155 forms the angles in fp32 (position * inv_freq) before cos/sin."""
    import numpy as np
    pos = torch.tensor([0, 1, 2, 77, 4095, 70000])
    c, s = orope.rope_cos_sin(pos, dtype=torch.float32)
    # inv_freq as model.py:145 computes it (torch's fp32 pow); numpy's pow may differ by an ulp
    inv = (1.0 / (1_000_000.0 ** (torch.arange(0, D, 2).float() / D))).numpy()
    ang = (pos.numpy().astype(np.float32)[:, None] * inv[None, :]).astype(np.float32)
    ang = np.concatenate([ang, ang], axis=1).astype(np.float64)
    assert np.abs(c.numpy() - np.cos(ang)).max() < 1e-6
    assert np.abs(s.numpy() - np.sin(ang)).max() < 1e-6
    assert torch.all(c[0] == 1) and torch.all(s[0] == 0)


def test_planted_sign_mistake_is_caught():
    x = torch.randn(8, 2, D, dtype=torch.float64)
    c, s = orope.rope_cos_sin(torch.arange(8) * 37, dtype=torch.float64)
    good = orope.apply_rope(x, c[:, None], s[:, None])
    wrong = x * c[:, None] + torch.cat((x[..., 64:], -x[..., :64]), dim=-1) * s[:, None]
    assert (good - wrong).abs().max() > 0.1


def test_cache_write_places_rows():
    pool = torch.zeros(10, 2, D)
    rows = torch.randn(3, 2, D)
    out = orope.cache_write(pool, torch.tensor([7, 0, 4], dtype=torch.int32), rows)
    assert torch.equal(out[7], rows[0]) and torch.equal(out[0], rows[1]) and torch.equal(out[4], rows[2])
    assert out[[1, 2, 3, 5, 6, 8, 9]].abs().sum() == 0


# --- the HIP kernel (GPU), bitwise against the oracle ------------------------------------------

def _case(n, dtype, seed, num_slots=64, row_pad=0, bad_slot=False):
    g = torch.Generator().manual_seed(seed)
    width = (N_Q + 2 * N_KV) * D
    big = torch.randn(n, width + row_pad, generator=g).to(dtype)
    qkv = big[:, :width]  # rows strided when row_pad > 0
    pos = torch.randint(0, 50000, (n,), generator=g)
    cos, sin = orope.rope_cos_sin(pos, dtype=dtype)
    slots = torch.randperm(num_slots, generator=g)[:n].to(torch.int32)
    if bad_slot:
        slots[n // 2] = num_slots + 3
    k_pool = torch.randn(num_slots, N_KV, D, generator=g).to(dtype)
    v_pool = torch.randn(num_slots, N_KV, D, generator=g).to(dtype)
    return qkv, cos, sin, slots, k_pool, v_pool


def _oracle(qkv, cos, sin, slots, k_pool, v_pool):
    n = qkv.shape[0]
    x = qkv.reshape(n, N_Q + 2 * N_KV, D)
    q = orope.apply_rope(x[:, :N_Q], cos[:, None], sin[:, None])
    k = orope.apply_rope(x[:, N_Q:N_Q + N_KV], cos[:, None], sin[:, None])
    v = x[:, N_Q + N_KV:]
    ok = (slots >= 0) & (slots < k_pool.shape[0])
    return (q.reshape(n, N_Q * D), orope.cache_write(k_pool, slots[ok], k[ok]),
            orope.cache_write(v_pool, slots[ok], v[ok]))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("n,row_pad,bad", [(1, 0, False), (7, 0, False), (300, 64, False),
                                           (40, 0, True)], ids=["1", "7", "300-strided", "bad-slot"])
def test_rope_kv_write_is_bitwise_the_oracle(dtype, n, row_pad, bad):
    from kernels.rope import rope_kv_write
    qkv, cos, sin, slots, kp, vp = _case(n, dtype, seed=n, num_slots=max(64, 2 * n),
                                         row_pad=row_pad, bad_slot=bad)
    q_want, k_want, v_want = _oracle(qkv, cos, sin, slots, kp, vp)
    announce(f"[gpu] rope_kv_write n={n} {dtype} pad={row_pad} bad={bad}")
    kp_d, vp_d = kp.cuda(), vp.cuda()
    q_out = rope_kv_write(qkv.cuda(), cos.cuda(), sin.cuda(), slots.cuda(), kp_d, vp_d, N_Q, N_KV)
    torch.cuda.synchronize()
    assert torch.equal(q_out.cpu(), q_want)
    assert torch.equal(kp_d.cpu(), k_want)
    assert torch.equal(vp_d.cpu(), v_want)


@pytest.mark.gpu
def test_rope_kv_write_matches_the_torch_gpu_path():
    """Same as the model's unfused GPU code (apply_rope + index_copy_ on the device)."""
    from kernels.rope import rope_kv_write
    qkv, cos, sin, slots, kp, vp = _case(33, torch.bfloat16, seed=5)
    qkv, cos, sin, slots, kp, vp = (t.cuda() for t in (qkv, cos, sin, slots, kp, vp))
    x = qkv.reshape(33, N_Q + 2 * N_KV, D)
    q_t = orope.apply_rope(x[:, :N_Q], cos[:, None], sin[:, None]).reshape(33, -1)
    k_t = orope.apply_rope(x[:, N_Q:N_Q + N_KV], cos[:, None], sin[:, None])
    kp_t, vp_t = kp.clone(), vp.clone()
    kp_t.index_copy_(0, slots.long(), k_t)
    vp_t.index_copy_(0, slots.long(), x[:, N_Q + N_KV:].contiguous())
    announce("[gpu] rope_kv_write vs torch on the device")
    q_out = rope_kv_write(qkv, cos, sin, slots, kp, vp, N_Q, N_KV)
    torch.cuda.synchronize()
    assert torch.equal(q_out, q_t) and torch.equal(kp, kp_t) and torch.equal(vp, vp_t)

"""CPU restatement of the step before attention: rotary embedding and the paged cache write.
TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

  rotate_half / apply_rope  model.py:58-65 (applied at model.py:92): q*cos + rotate_half(q)*sin in
                            the tensor dtype, each op rounding as torch's 16-bit ops do.
  rope_cos_sin              model.py:151-155: cos/sin tables of the positions, in the dtype.
  cache_write               kv_cache.py:108-115: this step's k/v rows into their cache slots.
"""
import torch


def rotate_half(x):
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


def apply_rope(x, cos, sin):
    """x [..., 128], cos/sin broadcastable, all in the same dtype."""
    return x * cos + rotate_half(x) * sin


def rope_cos_sin(positions, head_dim=128, theta=1_000_000.0, dtype=torch.bfloat16):
    """positions [n] -> cos, sin [n, head_dim]."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))
    freqs = positions.float()[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def cache_write(pool, slots, rows):
    """pool [slots, heads, d]; rows [n, heads, d] written at pool[slots[i]]."""
    out = pool.clone()
    out.index_copy_(0, slots.long(), rows)
    return out

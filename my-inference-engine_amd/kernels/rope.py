"""Fused rotary embedding + paged KV-cache write (the step before attention), on the HIP kernel.

`rope_kv_write` replaces, on the GPU path, the reference's apply_rope (model.py:62-65, applied at
model.py:92) followed by KVCache.write (kv_cache.py:108-115, called at model.py:96): one launch per
layer reads each new token's fused q|k|v projection row, rotates q and k with the model's cos/sin
tables, returns the rotated q and scatters the rotated k and the v into the token's cache slot.
The results are bitwise those of the unfused torch code (same 16-bit rounding after each multiply
and after the add).  No CPU path: CPU tensors are rejected.
"""
import torch

from . import _lib

HEAD_DIM = 128


def rope_kv_write(qkv, cos, sin, slot_mapping, k_pool, v_pool, heads_q, heads_kv, q_out=None):
    """qkv [n, (heads_q + 2*heads_kv)*128] (rows may be strided), cos/sin [n, 128], slot_mapping
    [n] int32, k_pool/v_pool [slots, heads_kv, 128] (one layer of KVCache.buf).

    Returns q_out [n, heads_q*128], the rotated queries (allocated unless given)."""
    assert qkv.is_cuda and cos.is_cuda and sin.is_cuda and k_pool.is_cuda and v_pool.is_cuda, \
        "rope_kv_write runs on the GPU only"
    assert qkv.dtype in _lib.DTYPES and cos.dtype == qkv.dtype and sin.dtype == qkv.dtype
    assert k_pool.dtype == qkv.dtype and v_pool.dtype == qkv.dtype
    n = qkv.shape[0]
    assert qkv.dim() == 2 and qkv.stride(1) == 1 and qkv.shape[1] == (heads_q + 2 * heads_kv) * HEAD_DIM
    assert cos.shape == (n, HEAD_DIM) and sin.shape == (n, HEAD_DIM) and cos.stride() == sin.stride()
    assert cos.stride(1) == 1
    assert slot_mapping.dtype == torch.int32 and slot_mapping.shape == (n,) and slot_mapping.is_contiguous()
    assert k_pool.dim() == 3 and k_pool.shape == v_pool.shape and k_pool.stride() == v_pool.stride()
    assert k_pool.shape[1:] == (heads_kv, HEAD_DIM) and k_pool.stride(2) == 1
    if q_out is None:
        q_out = torch.empty(n, heads_q * HEAD_DIM, device=qkv.device, dtype=qkv.dtype)
    assert q_out.shape == (n, heads_q * HEAD_DIM) and q_out.stride(1) == 1
    lib = _lib.load()
    pool_strides = (_lib.ctypes.c_int64 * 2)(*k_pool.stride()[:2])
    _lib.check(lib.mi_fa2_rope_kv_write(
        _lib.DTYPES[qkv.dtype], qkv.data_ptr(), qkv.stride(0), cos.data_ptr(), sin.data_ptr(),
        cos.stride(0), slot_mapping.data_ptr(), n, heads_q, heads_kv, HEAD_DIM, q_out.data_ptr(),
        q_out.stride(0), k_pool.data_ptr(), v_pool.data_ptr(), pool_strides, k_pool.shape[0],
        _lib.stream_of(qkv)))
    return q_out

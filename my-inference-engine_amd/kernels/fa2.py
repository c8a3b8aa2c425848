"""FlashAttention-2 forward on MI355X: drop-in for the reference's kernels/fa2.py.

`FlashAttention2Function.apply(Q, K, V, is_causal=False, kv_lens=None) -> O` keeps the call
signature, argument meaning, checks (AssertionError) and outputs of kernels/fa2.py:164-214, so the
reference's model.py:11-15,102-103 import and call it unchanged.  The Triton launch
(kernels/fa2.py:192-207) is replaced by one call into libmi_fa2.so's C ABI, which runs hand-written
gfx950 kernels on torch's current stream:

  * seqlen_q > 1: the MFMA prefill kernel (csrc/fa2_prefill.hip);
  * seqlen_q == 1: the split-KV decode kernel + combine (csrc/fa2_decode.hip);
  * any other head dims (powers of two from 16 to 256, d_v may differ from d) or fp32 inputs: the
    general kernel (csrc/fa2_general.hip), for every seqlen_q.

Three entry points go beyond the reference's padded call:

  * `fa2_paged(q, k_pool, v_pool, block_table, kv_lens, ...)` reads K/V straight out of a
    KVCache-layout pool (kv_cache.py:20-22) through a block table, replacing
    KVCache.read's per-step dense gather (kv_cache.py:117-121) + the padded call.
  * `fa2_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, is_causal)` runs a ragged
    batch packed back to back (no padding).
  * `fa2_paged_varlen(q, k_pool, v_pool, cu_seqlens_q, block_table, kv_lens, max_seqlen_q, ...)`
    runs packed rows with different new-token counts over the paged pool in one launch (the
    prompts of a mixed prefill + decode step).

The paged and packed entry points cover head_dim 128 in bf16/fp16 (the Qwen2.5-1.5B shape the
engine runs); the padded call also takes the rest of the reference's envelope (kernels/fa2.py:185:
power-of-two d and d_v; fp32 inputs with fp32 dots, kernels/fa2.py:129,147) up to 256.  Anything
else is rejected with an AssertionError, never silently computed another way.
"""
import math

import torch

from . import _lib

HEAD_DIM = 128


_MEMO_MAX = 4096
_STRIDES_OK = {}
_STRIDE_ARRAYS = {}


def _strides_ok(t):
    """Strides that allow 16-byte vector loads (the base alignment is checked per call)."""
    key = (t.shape, t.stride())
    ok = _STRIDES_OK.get(key)
    if ok is None:
        shape, stride = key
        ok = stride[-1] == 1 and all(st % 8 == 0 for st, n in zip(stride[:-1], shape[:-1]) if n > 1)
        if len(_STRIDES_OK) >= _MEMO_MAX:
            _STRIDES_OK.clear()
        _STRIDES_OK[key] = ok
    return ok


def _dims_ok(t):
    return t.data_ptr() % 16 == 0 and _strides_ok(t)


def _vec(t):
    """t, or a contiguous copy if its layout does not allow 16-byte vector loads."""
    return t if _dims_ok(t) else t.contiguous()


def _contig(shape):
    return tuple(math.prod(shape[i + 1:]) for i in range(len(shape)))


def _strides_of(shape, stride):
    # A size-1 dimension is only ever indexed at 0, so its stride never moves an address, and torch
    # may report any value there (0 after expand, anything after a view).  The kernels also use a
    # token stride as the row pitch of their load extents (a load of `rows` rows reads at most
    # rows * stride elements from the first row's start), so a size-1 dimension gets the stride it
    # would have in a contiguous tensor: the product of the sizes after it, never less than the
    # head dim.  (A 0 there made a single-token K or V read as zeros.)
    # The arrays are memoised by (shape, stride): the C ABI only reads them.
    key = (tuple(shape), tuple(stride))
    arr = _STRIDE_ARRAYS.get(key)
    if arr is None:
        s = [math.prod(shape[i + 1:]) if n == 1 else st
             for i, (st, n) in enumerate(zip(stride, shape))]
        arr = (_lib.ctypes.c_int64 * len(s))(*s)
        if len(_STRIDE_ARRAYS) >= _MEMO_MAX:
            _STRIDE_ARRAYS.clear()
        _STRIDE_ARRAYS[key] = arr
    return arr


def _strides(t):
    return _strides_of(t.shape, t.stride())


_POOL_STRIDES = {}


def _pool_strides(pool):
    """(slot, head) strides of a [slots, Hkv, d] pool, as they are."""
    key = pool.stride()[:2]
    arr = _POOL_STRIDES.get(key)
    if arr is None:
        arr = (_lib.ctypes.c_int64 * 2)(*key)
        if len(_POOL_STRIDES) >= _MEMO_MAX:
            _POOL_STRIDES.clear()
        _POOL_STRIDES[key] = arr
    return arr


GENERAL_DIMS = (16, 32, 64, 128, 256)


def _general_envelope(Q, K, V):
    """The general kernel's envelope: bf16/fp16/fp32, power-of-two d and d_v from 16 to 256."""
    assert Q.dtype in _lib.GENERAL_DTYPES, \
        f"the MI355X kernels take bf16, fp16 or fp32 inputs, got {Q.dtype}"
    assert K.dtype == Q.dtype and V.dtype == Q.dtype, "Q, K and V must share one dtype"
    assert Q.shape[-1] in GENERAL_DIMS and V.shape[-1] in GENERAL_DIMS, (
        f"the MI355X kernels take head dims 16 to 256, got d={Q.shape[-1]}, d_v={V.shape[-1]}")
    assert K.device == Q.device and V.device == Q.device, "Q, K and V must be on one device"
    assert Q.shape[0] <= 65535 and Q.shape[1] <= 65535, "batch and heads are at most 65535"


def _envelope(Q, K, V):
    assert Q.dtype in _lib.DTYPES, f"the MI355X kernels take bf16 or fp16 inputs, got {Q.dtype}"
    assert K.dtype == Q.dtype and V.dtype == Q.dtype, "Q, K and V must share one dtype"
    assert Q.shape[-1] == HEAD_DIM and V.shape[-1] == HEAD_DIM, (
        f"the MI355X kernels are built for head_dim {HEAD_DIM}, got d={Q.shape[-1]}, d_v={V.shape[-1]}")
    assert K.device == Q.device and V.device == Q.device, "Q, K and V must be on one device"


_WORKSPACES = {}
_RETIRED = []   # outgrown workspaces: never freed (a captured graph may still use one)


def _workspace(nbytes, device):
    """The split-decode workspace of (device, current stream), grown on demand.

    Its contents need no initialisation (every partial the combine reads is written by the same
    launch), so it is allocated uninitialised -- no fill, which also keeps a captured graph free of
    memset nodes; one buffer per stream keeps calls on different streams from sharing it.  A
    buffer that is outgrown is kept alive, not freed: a HIP graph captured with it holds its
    address, and torch keeps alive only the memory a capture itself allocated."""
    if not nbytes:
        return None
    key = (device, torch._C._cuda_getCurrentRawStream(_lib.device_index(device)))
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        size = int(nbytes)
        if ws is not None:
            _RETIRED.append(ws)
            # at least double: a workspace that grows step by step (one split more every 128
            # keys of a growing row) retires O(log) buffers whose sizes sum to less than its own
            size = max(size, 2 * ws.numel())
        ws = torch.empty(size, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


class _Padded:
    """The validated launch of one padded-call shape: its checks ran once, its constant arguments
    (sizes, stride arrays, output shapes, which kernel) are built once, and every later call of the
    same shapes, strides, dtypes, device and causality only allocates O and L and launches.

    Checked per call, not cached: tensor base alignment (16 bytes) and kv_lens."""
    __slots__ = ("fast", "dtype_code", "dev", "o_shape", "l_shape", "copy_q", "copy_k", "copy_v",
                 "head", "tail", "ws_bytes")


_PADDED = {}
_MEMO_MAX = 4096


def _plan_padded(Q, K, V, is_causal):
    """Every check of FlashAttention2Function.forward (kernels/fa2.py:172-185), then the launch's
    constant arguments."""
    batch_size, num_heads, seq_len, d = Q.shape
    seq_len_k = K.shape[2]
    d_v = V.shape[-1]
    sm_scale = 1.0 / math.sqrt(d)
    assert Q.is_cuda and K.is_cuda and V.is_cuda, "Q, K and V must be GPU tensors"
    num_kv_heads = K.shape[1]
    assert Q.shape[0] == K.shape[0] and Q.shape[-1] == K.shape[-1], \
        "Q and K must agree in batch size and head dim"
    assert num_heads % num_kv_heads == 0, "query heads must be a multiple of kv heads (GQA)"
    assert K.shape[:-1] == V.shape[:-1], "K and V may differ only in their last dimension"
    assert (d & (d - 1) == 0) and (d_v & (d_v - 1) == 0), "d and d_v must be powers of 2"
    fast = Q.dtype in _lib.DTYPES and d == HEAD_DIM and d_v == HEAD_DIM
    if fast:
        _envelope(Q, K, V)
    else:
        _general_envelope(Q, K, V)
    pl = _Padded()
    pl.fast = fast
    pl.dtype_code = (_lib.DTYPES if fast else _lib.GENERAL_DTYPES)[Q.dtype]
    pl.dev = Q.device
    pl.o_shape = (batch_size, num_heads, seq_len, d_v)
    pl.l_shape = (batch_size, num_heads, seq_len)
    # a tensor whose strides do not allow 16-byte vector loads goes through a contiguous copy
    pl.copy_q, pl.copy_k, pl.copy_v = (not _strides_ok(t) for t in (Q, K, V))
    lay = lambda t, cp: _strides_of(t.shape, _contig(t.shape) if cp else t.stride())  # noqa: E731
    o_st = _strides_of(pl.o_shape, _contig(pl.o_shape))
    l_st = _strides_of(pl.l_shape, _contig(pl.l_shape))
    qs, ks, vs = lay(Q, pl.copy_q), lay(K, pl.copy_k), lay(V, pl.copy_v)
    if fast:
        pl.head = (batch_size, num_heads, num_kv_heads, seq_len, seq_len_k, d)
        pl.tail = (qs, ks, vs, o_st, l_st, int(bool(is_causal)), sm_scale)
        pl.ws_bytes = _lib.load().mi_fa2_fwd_workspace_size(batch_size, num_heads, num_kv_heads,
                                                             seq_len, seq_len_k, d)
    else:
        pl.head = (batch_size, num_heads, num_kv_heads, seq_len, seq_len_k, d, d_v)
        pl.tail = (qs, ks, vs, o_st, l_st, int(bool(is_causal)), sm_scale)
        pl.ws_bytes = 0
    return pl


def _run_padded(Q, K, V, is_causal, kv_lens, want_lse=True):
    """The padded forward: (O, L), launched on the current stream of Q's device.  want_lse=False
    skips L (None is returned in its place): the kernels then store no LSE."""
    key = (Q.shape, Q.stride(), K.shape, K.stride(), V.shape, V.stride(), Q.dtype, K.dtype,
           V.dtype, Q.device, K.device, V.device, bool(is_causal))
    pl = _PADDED.get(key)
    if pl is None:
        pl = _plan_padded(Q, K, V, is_causal)
        if len(_PADDED) >= _MEMO_MAX:
            _PADDED.clear()
        _PADDED[key] = pl
    if kv_lens is not None:
        assert kv_lens.shape == (pl.o_shape[0],) and kv_lens.dtype == torch.int32, \
            "kv_lens must be an int32 tensor of shape [batch]"
        assert kv_lens.device == Q.device, "kv_lens must be on Q's device"
    q = Q.contiguous() if pl.copy_q else Q
    k = K.contiguous() if pl.copy_k else K
    v = V.contiguous() if pl.copy_v else V
    tail = pl.tail
    if (q.data_ptr() | k.data_ptr() | v.data_ptr()) & 15:
        # a view starting off a 16-byte boundary: an aligned copy (.contiguous() would return an
        # already-contiguous view as it is), launched with the copies' own strides
        q, k, v = (t.clone(memory_format=torch.contiguous_format) if t.data_ptr() & 15 else t
                   for t in (q, k, v))
        tail = (_strides(q), _strides(k), _strides(v)) + tail[3:]
    dev = pl.dev
    O = torch.empty(pl.o_shape, device=dev, dtype=Q.dtype)
    L = torch.empty(pl.l_shape, device=dev, dtype=torch.float32) if want_lse else None
    lp = L.data_ptr() if want_lse else None
    lib = _lib.load()
    lens = kv_lens.data_ptr() if kv_lens is not None else None
    with _lib.on_device(dev) as stream:
        if pl.fast:
            ws = _workspace(pl.ws_bytes, dev)
            _lib.check(lib.mi_fa2_fwd(
                pl.dtype_code, q.data_ptr(), k.data_ptr(), v.data_ptr(), O.data_ptr(),
                lp, lens, *pl.head, *tail,
                ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
                stream))
        else:
            _lib.check(lib.mi_fa2_fwd_general(
                pl.dtype_code, q.data_ptr(), k.data_ptr(), v.data_ptr(), O.data_ptr(),
                lp, lens, *pl.head, *tail, stream))
    return O, L


class FlashAttention2Function(torch.autograd.Function):
    @staticmethod
    def forward(ctx, Q, K, V, is_causal=False, kv_lens=None):
        # Q [B, Hq, T, d], K/V [B, Hkv, S, d]; kv_lens [B] int32: real keys per row (the rest of
        # K/V is padding); causal masking is aligned to each row's last key.
        O, L = _run_padded(Q, K, V, is_causal, kv_lens)
        ctx.save_for_backward(Q, K, V, O, L)
        ctx.is_causal = is_causal
        ctx.scale = 1.0 / math.sqrt(Q.shape[-1])
        return O

    @classmethod
    def apply(cls, Q, K, V, is_causal=False, kv_lens=None):
        """Same call and result as torch.autograd.Function.apply.  The reference's Function has a
        forward only (kernels/fa2.py:164-214): an autograd node is recorded when an input
        requires grad, as before, and L is saved on it; otherwise (inference, every call of the
        engine) no node exists to save L on, so the forward runs directly and computes O alone,
        without the node machinery's host cost (several microseconds per call)."""
        if torch.is_grad_enabled() and (Q.requires_grad or K.requires_grad or V.requires_grad):
            return super().apply(Q, K, V, is_causal, kv_lens)
        return _run_padded(Q, K, V, is_causal, kv_lens, want_lse=False)[0]


def fa2_forward(Q, K, V, is_causal=False, kv_lens=None, return_lse=False):
    """Functional form of FlashAttention2Function.apply; optionally also returns the fp32 LSE."""
    if not return_lse:
        return FlashAttention2Function.apply(Q, K, V, is_causal, kv_lens)
    with torch.no_grad():
        ctx = _Ctx()
        O = FlashAttention2Function.forward(ctx, Q, K, V, is_causal, kv_lens)
    return O, ctx.saved[4]


class _Ctx:
    def save_for_backward(self, *t):
        self.saved = t


def fa2_paged(q, k_pool, v_pool, block_table, kv_lens, *, block_size=16, max_kv_len=None,
              is_causal=None, out=None, return_lse=False):
    """Attention over K/V held in a paged pool, read in-kernel through a block table.

    q            [B, Hq, T, 128]   this step's queries (T = 1 for decode)
    k_pool/v_pool [num_blocks*block_size, Hkv, 128]: one layer of KVCache.buf (kv_cache.py:20-22)
    block_table  [B, W] int32: row b's token p is at slot block_table[b, p // block_size] *
                 block_size + p % block_size (kv_cache.py:15-16)
    kv_lens      [B] int32: keys per row including this step's T (model.py:175)
    max_kv_len   host-side upper bound of kv_lens (default W * block_size)
    is_causal    default T > 1, as model.py:185 sets it; bottom-right aligned per row
    out          optional [B, Hq, T, 128] output (any row/head/token strides, 16-byte aligned)
    Returns O [B, Hq, T, 128] (and the fp32 LSE [B, Hq, T] if return_lse).
    """
    assert q.is_cuda and k_pool.is_cuda and v_pool.is_cuda, "q and the pools must be GPU tensors"
    B, Hq, T, d = q.shape
    assert k_pool.dim() == 3 and k_pool.shape == v_pool.shape, "pools are [slots, Hkv, d]"
    assert k_pool.stride() == v_pool.stride(), "k_pool and v_pool must share strides"
    Hkv = k_pool.shape[1]
    assert Hq % Hkv == 0, "query heads must be a multiple of kv heads (GQA)"
    assert block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.shape[0] == B
    assert kv_lens.dtype == torch.int32 and kv_lens.shape == (B,)
    assert block_table.stride(-1) == 1, "block_table rows must be contiguous"
    assert block_size >= 16 and block_size & (block_size - 1) == 0, "block_size: power of 2, >= 16"
    assert k_pool.shape[0] % block_size == 0, "pool slots must be whole blocks"
    _envelope(q, k_pool, v_pool)
    if max_kv_len is None:
        max_kv_len = block_table.shape[1] * block_size
    # kv_lens are clamped to max_kv_len in-kernel, so this bound keeps every table read in range
    assert 0 <= max_kv_len <= block_table.shape[1] * block_size, \
        "max_kv_len exceeds what the block table can address"
    if is_causal is None:
        is_causal = T > 1
    q = _vec(q)
    assert _dims_ok(k_pool) and _dims_ok(v_pool), "pools need 16-byte aligned token rows"
    O = out if out is not None else torch.empty((B, Hq, T, d), device=q.device, dtype=q.dtype)
    assert O.shape == q.shape and O.dtype == q.dtype and _dims_ok(O)
    L = torch.empty((B, Hq, T), device=q.device, dtype=torch.float32) if return_lse else None
    lib = _lib.load()
    ws = _workspace(_paged_ws_bytes(B, Hq, Hkv, T, int(max_kv_len), d), q.device)
    pool_strides = _pool_strides(k_pool)
    with _lib.on_device(q.device) as stream:
        _lib.check(lib.mi_fa2_fwd_paged(
            _lib.DTYPES[q.dtype], q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), O.data_ptr(),
            L.data_ptr() if L is not None else None, block_table.data_ptr(), block_table.stride(0),
            kv_lens.data_ptr(), B, Hq, Hkv, T, int(max_kv_len), d, block_size,
            k_pool.shape[0] // block_size, _strides(q), pool_strides, _strides(O),
            _strides(L) if L is not None else None, int(bool(is_causal)),
            1.0 / math.sqrt(d), ws.data_ptr() if ws is not None else None,
            ws.numel() if ws is not None else 0, stream))
    return (O, L) if return_lse else O


_WS_BYTES = {}


def _paged_ws_bytes(*dims):
    n = _WS_BYTES.get(dims)
    if n is None:
        n = _lib.load().mi_fa2_fwd_paged_workspace_size(*dims)
        if len(_WS_BYTES) >= _MEMO_MAX:
            _WS_BYTES.clear()
        _WS_BYTES[dims] = n
    return n


def fa2_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, is_causal=False,
               return_lse=False, out=None):
    """Attention over a ragged batch packed back to back.

    q [total_q, Hq, 128], k/v [total_k, Hkv, 128]; cu_seqlens_q/k [B+1] int32 prefix offsets;
    row b = q[cu_q[b]:cu_q[b+1]] against k/v[cu_k[b]:cu_k[b+1]], causal aligned to the row's end.
    out: optional [total_q, Hq, 128] output (any token/head strides, 16-byte aligned).
    Returns O [total_q, Hq, 128] (and the fp32 LSE [Hq, total_q] if return_lse).
    """
    assert q.is_cuda and k.is_cuda and v.is_cuda, "q, k and v must be GPU tensors"
    assert q.dim() == 3 and k.dim() == 3 and k.shape[:-1] == v.shape[:-1]
    assert cu_seqlens_q.dtype == torch.int32 and cu_seqlens_k.dtype == torch.int32
    B = cu_seqlens_q.shape[0] - 1
    assert cu_seqlens_k.shape[0] == B + 1
    total_q, Hq, d = q.shape
    Hkv = k.shape[1]
    assert Hq % Hkv == 0, "query heads must be a multiple of kv heads (GQA)"
    _envelope(q, k, v)
    q, k, v = _vec(q), _vec(k), _vec(v)
    O = out if out is not None else torch.empty((total_q, Hq, d), device=q.device, dtype=q.dtype)
    assert O.shape == q.shape and O.dtype == q.dtype and _dims_ok(O)
    L = torch.empty((Hq, total_q), device=q.device, dtype=torch.float32) if return_lse else None
    lib = _lib.load()
    with _lib.on_device(q.device) as stream:
        _lib.check(lib.mi_fa2_fwd_varlen(
            _lib.DTYPES[q.dtype], q.data_ptr(), k.data_ptr(), v.data_ptr(), O.data_ptr(),
            L.data_ptr() if L is not None else None, cu_seqlens_q.data_ptr(),
            cu_seqlens_k.data_ptr(), B, Hq, Hkv, int(max_seqlen_q), d, _strides(q), _strides(k),
            _strides(v), _strides(O), _strides(L) if L is not None else None,
            int(bool(is_causal)), 1.0 / math.sqrt(d), stream))
    return (O, L) if return_lse else O


def fa2_paged_varlen(q, k_pool, v_pool, cu_seqlens_q, block_table, kv_lens, max_seqlen_q, *,
                     block_size=16, max_kv_len=None, is_causal=True, out=None, return_lse=False):
    """Packed prefill of several rows over the paged cache, one launch.

    q            [total_q, Hq, 128]: row b's new queries are q[cu_q[b]:cu_q[b+1]] (rows may have
                 different counts, 0 included)
    k_pool/v_pool, block_table, kv_lens, block_size, max_kv_len: as in fa2_paged; kv_lens include
                 each row's new tokens, whose K/V are already in the pool
    is_causal    bottom-right aligned per row (query i of row b sees keys <= i + kv_len - T_b)
    out          optional [total_q, Hq, 128] output (any token/head strides)
    Returns O [total_q, Hq, 128] (and the fp32 LSE [Hq, total_q] if return_lse).
    """
    assert q.is_cuda and k_pool.is_cuda and v_pool.is_cuda, "q and the pools must be GPU tensors"
    assert q.dim() == 3, "q is [total_q, Hq, d]"
    total_q, Hq, d = q.shape
    B = cu_seqlens_q.shape[0] - 1
    assert k_pool.dim() == 3 and k_pool.shape == v_pool.shape, "pools are [slots, Hkv, d]"
    assert k_pool.stride() == v_pool.stride(), "k_pool and v_pool must share strides"
    Hkv = k_pool.shape[1]
    assert Hq % Hkv == 0, "query heads must be a multiple of kv heads (GQA)"
    assert cu_seqlens_q.dtype == torch.int32 and kv_lens.dtype == torch.int32
    assert kv_lens.shape == (B,)
    assert block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.shape[0] == B
    assert block_table.stride(-1) == 1, "block_table rows must be contiguous"
    assert block_size >= 16 and block_size & (block_size - 1) == 0, "block_size: power of 2, >= 16"
    assert k_pool.shape[0] % block_size == 0, "pool slots must be whole blocks"
    _envelope(q, k_pool, v_pool)
    if max_kv_len is None:
        max_kv_len = block_table.shape[1] * block_size
    assert 0 <= max_kv_len <= block_table.shape[1] * block_size, \
        "max_kv_len exceeds what the block table can address"
    q = _vec(q)
    assert _dims_ok(k_pool) and _dims_ok(v_pool), "pools need 16-byte aligned token rows"
    O = out if out is not None else torch.empty((total_q, Hq, d), device=q.device, dtype=q.dtype)
    assert O.shape == q.shape and O.dtype == q.dtype and _dims_ok(O)
    L = torch.empty((Hq, total_q), device=q.device, dtype=torch.float32) if return_lse else None
    lib = _lib.load()
    pool_strides = _pool_strides(k_pool)
    with _lib.on_device(q.device) as stream:
        _lib.check(lib.mi_fa2_fwd_paged_varlen(
            _lib.DTYPES[q.dtype], q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), O.data_ptr(),
            L.data_ptr() if L is not None else None, cu_seqlens_q.data_ptr(),
            block_table.data_ptr(), block_table.stride(0), kv_lens.data_ptr(), B, Hq, Hkv,
            int(max_seqlen_q), int(max_kv_len), d, block_size, k_pool.shape[0] // block_size,
            _strides(q), pool_strides, _strides(O), _strides(L) if L is not None else None,
            int(bool(is_causal)), 1.0 / math.sqrt(d), stream))
    return (O, L) if return_lse else O


_OUT_DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def fa2_combine(part_o, part_lse, n_parts=None, out_dtype=torch.bfloat16, return_lse=False):
    """Merge attention partials computed over disjoint key ranges (mi_fa2_combine).

    part_o   [P, R, H, 128] fp32: partial i of (row r, head h) is the normalised output of a
             forward over a sub-range of the row's keys
    part_lse [P, R, H] fp32: its log-sum-exp (natural log, the L of kernels/fa2.py:155-158);
             -inf: the partial saw no key (its O is not read)
    n_parts  [R] int32: partials used per row (the first n_parts[r]), or None: all P
    Returns O [R, H, 128] in out_dtype (and the merged fp32 lse [R, H] if return_lse): what one
    pass over all the keys gives.
    """
    assert part_o.is_cuda and part_lse.is_cuda, "partials must be GPU tensors"
    assert part_o.dtype == torch.float32 and part_lse.dtype == torch.float32
    assert part_o.dim() == 4 and part_o.shape[-1] == HEAD_DIM and part_o.stride(-1) == 1
    P, R, H, d = part_o.shape
    assert part_lse.shape == (P, R, H), "part_lse is [parts, rows, heads]"
    assert out_dtype in _OUT_DTYPES, f"out_dtype must be bf16, fp16 or fp32, got {out_dtype}"
    if n_parts is not None:
        assert n_parts.dtype == torch.int32 and n_parts.shape == (R,) and n_parts.is_contiguous()
        assert n_parts.device == part_o.device
    if part_o.data_ptr() % 8:
        # a fresh allocation: .contiguous() would hand back an already-contiguous view as it is,
        # still misaligned for the kernel's paired 8-byte loads
        part_o = part_o.clone(memory_format=torch.contiguous_format)
    elif any(st % 2 for st in part_o.stride()[:-1]):
        part_o = part_o.contiguous()
    O = torch.empty((R, H, d), device=part_o.device, dtype=out_dtype)
    L = torch.empty((R, H), device=part_o.device, dtype=torch.float32) if return_lse else None
    lib = _lib.load()
    with torch.cuda.device(part_o.device):
        _lib.check(lib.mi_fa2_combine(
            _OUT_DTYPES[out_dtype], part_o.data_ptr(), part_lse.data_ptr(),
            n_parts.data_ptr() if n_parts is not None else None, R, H, P, d,
            _lib.strides(part_o, 3), _lib.strides(part_lse, 3), O.data_ptr(), _lib.strides(O, 2),
            L.data_ptr() if L is not None else None, _lib.strides(L, 2) if L is not None else None,
            _lib.stream_of(part_o)))
    return (O, L) if return_lse else O

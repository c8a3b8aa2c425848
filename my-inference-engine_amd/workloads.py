"""Seeded synthetic inputs of the attention workloads (CPU tensors; callers move them to the GPU).

All values come from torch.Generator().manual_seed(seed) on the CPU, so a CPU check and a GPU run
see bit-identical inputs.  Shapes are Qwen2.5-1.5B's attention: 12 query heads over 2 kv heads,
head_dim 128 (model.py:18-23), paged KV in 16-token blocks (chat.py:22).
"""
import math

import torch

NUM_HEADS = 12
NUM_KV_HEADS = 2
HEAD_DIM = 128
BLOCK_SIZE = 16


def prefill_single(seq_len=4096, dtype=torch.bfloat16, seed=0, heads=NUM_HEADS,
                   kv_heads=NUM_KV_HEADS):
    """One causal sequence: q [1, 12, L, 128], k/v [1, 2, L, 128] ~ N(0, 1)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, heads, seq_len, HEAD_DIM, generator=g).to(dtype)
    k = torch.randn(1, kv_heads, seq_len, HEAD_DIM, generator=g).to(dtype)
    v = torch.randn(1, kv_heads, seq_len, HEAD_DIM, generator=g).to(dtype)
    return q, k, v


def prefill_ragged(n_seqs=16, lo=16, hi=1024, dtype=torch.bfloat16, seed=0):
    """Packed varlen prefill: lengths ~ U[lo, hi], q [sum L, 12, 128], k/v [sum L, 2, 128].

    Returns (q, k, v, lens, cu_seqlens) with cu_seqlens a list of n_seqs + 1 offsets."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (n_seqs,), generator=g).tolist()
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    total = cu[-1]
    q = torch.randn(total, NUM_HEADS, HEAD_DIM, generator=g).to(dtype)
    k = torch.randn(total, NUM_KV_HEADS, HEAD_DIM, generator=g).to(dtype)
    v = torch.randn(total, NUM_KV_HEADS, HEAD_DIM, generator=g).to(dtype)
    return q, k, v, lens, cu


def decode_paged(n_rows=64, lo=128, hi=8192, block_size=BLOCK_SIZE, dtype=torch.bfloat16, seed=0,
                 spare_blocks=0):
    """Batched decode over a paged pool: kv_lens ~ U[lo, hi]; every row's blocks are drawn from a
    random permutation of the pool.

    Returns (q [n_rows, 12, 1, 128], k_pool, v_pool [num_blocks*bs, 2, 128], tables, kv_lens) where
    tables is a list of per-row block-id lists."""
    g = torch.Generator().manual_seed(seed)
    kv_lens = torch.randint(lo, hi + 1, (n_rows,), generator=g).tolist()
    need = [math.ceil(n / block_size) for n in kv_lens]
    num_blocks = sum(need) + spare_blocks
    perm = torch.randperm(num_blocks, generator=g).tolist()
    tables, at = [], 0
    for n in need:
        tables.append(perm[at:at + n])
        at += n
    q = torch.randn(n_rows, NUM_HEADS, 1, HEAD_DIM, generator=g).to(dtype)
    k_pool = torch.randn(num_blocks * block_size, NUM_KV_HEADS, HEAD_DIM, generator=g).to(dtype)
    v_pool = torch.randn(num_blocks * block_size, NUM_KV_HEADS, HEAD_DIM, generator=g).to(dtype)
    return q, k_pool, v_pool, tables, kv_lens


def prefill_paged(seq_len=4096, block_size=BLOCK_SIZE, dtype=torch.bfloat16, seed=0):
    """One causal prompt whose keys sit in the paged pool, blocks in a random order: q
    [1, 12, L, 128], k_pool / v_pool [L, 2, 128] (exactly the prompt's blocks), its table."""
    g = torch.Generator().manual_seed(seed)
    n_blocks = math.ceil(seq_len / block_size)
    table = torch.randperm(n_blocks, generator=g).tolist()
    q = torch.randn(1, NUM_HEADS, seq_len, HEAD_DIM, generator=g).to(dtype)
    k_pool = torch.randn(n_blocks * block_size, NUM_KV_HEADS, HEAD_DIM, generator=g).to(dtype)
    v_pool = torch.randn(n_blocks * block_size, NUM_KV_HEADS, HEAD_DIM, generator=g).to(dtype)
    return q, k_pool, v_pool, [table]


def table_tensor(tables, width=None):
    """Per-row block lists -> [B, width] int32, short rows padded with block 0 (kv_cache.py:95)."""
    width = width if width is not None else max(1, max(len(t) for t in tables))
    return torch.tensor([(list(t) + [0] * width)[:width] for t in tables], dtype=torch.int32)


def causal_prefill_flops(lens, heads=NUM_HEADS, d=HEAD_DIM):
    """Algorithmic flops of causal attention: 4*d*heads per visible (query, key) pair."""
    return sum(4 * d * heads * n * (n + 1) // 2 for n in lens)


def decode_bytes(kv_lens, block_size=BLOCK_SIZE, heads=NUM_HEADS, kv_heads=NUM_KV_HEADS,
                 d=HEAD_DIM, elem=2):
    """Algorithmic HBM bytes of one paged decode step: every visible K and V element once, q and o
    once, the block-table entries covering each row and the row lengths."""
    kv = sum(kv_lens) * kv_heads * d * elem * 2
    qo = len(kv_lens) * heads * d * elem * 2
    table = sum(math.ceil(n / block_size) for n in kv_lens) * 4
    return kv + qo + table + 4 * len(kv_lens)

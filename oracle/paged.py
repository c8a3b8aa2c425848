"""Paged KV cache restatement (test infrastructure only; see oracle/__init__.py).

Restates the reference KVCache's slot arithmetic and per-step dense gather (kv_cache.py:15-16,
93-98, 117-121): logical token p of a row lives in slot table[p // block_size] * block_size +
p % block_size of a pool laid out [num_blocks * block_size, Hkv, d]; read() gathers every
position [0, S) of every row into a dense [B, Hkv, S, d] copy, positions past a row's table
pointing at block 0.
"""
import math

import torch


def slot_of(table_row, p, block_size):
    """Physical slot of logical token p (kv_cache.py:15-16)."""
    return table_row[p // block_size] * block_size + p % block_size


def gather_dense(pool, tables, S, block_size):
    """pool [P, Hkv, d], tables: list of per-row block-id lists -> dense [B, Hkv, S, d].

    Rows are padded with block 0 to ceil(S / block_size) blocks (kv_cache.py:93-95) and gathered
    with the index tables[b][pos // bs] * bs + pos % bs (kv_cache.py:96-98,117-121)."""
    n_blocks = math.ceil(S / block_size)
    padded = torch.tensor([(list(t) + [0] * n_blocks)[:n_blocks] for t in tables], dtype=torch.long)
    pos = torch.arange(S)
    gather_idx = padded[:, pos // block_size] * block_size + pos % block_size  # [B, S]
    return pool[gather_idx].transpose(1, 2)


def random_tables(kv_lens, block_size, num_blocks, generator):
    """Per-row block lists drawing distinct blocks from a random permutation of the pool."""
    need = [math.ceil(n / block_size) for n in kv_lens]
    assert sum(need) <= num_blocks, "pool too small for these rows"
    perm = torch.randperm(num_blocks, generator=generator).tolist()
    tables, at = [], 0
    for n in need:
        tables.append(perm[at:at + n])
        at += n
    return tables


def table_tensor(tables, width=None, fill=0):
    """Block lists -> [B, width] int32 (rows padded with `fill`)."""
    width = width if width is not None else max(1, max(len(t) for t in tables))
    return torch.tensor([(list(t) + [fill] * width)[:width] for t in tables], dtype=torch.int32)


def scatter_rows(k, kv_lens, tables, pool, block_size):
    """Write dense rows k [B, Hkv, S, d] (first kv_lens[b] tokens) into pool [P, Hkv, d]."""
    for b, n in enumerate(kv_lens):
        for p in range(n):
            pool[slot_of(tables[b], p, block_size)] = k[b, :, p]
    return pool

"""Per-step paged-cache metadata on the HIP kernel (csrc/step_meta.hip).

`step_metadata` replaces the host side of the reference's KVCache.prepare (kv_cache.py:74-101):
from the rows' sequence slots (and packed offsets) and the cache's device-resident tables and
lengths it writes starts, kv_lens, the batch block table, every new token's cache slot and,
optionally, positions and last indices, and advances the device lengths in place.  One launch on
the current stream; graph-capturable.  No CPU path.
"""
import torch

from . import _lib


def step_metadata(cache, row_slots, cu, tokens_per_row, starts, kv_lens, block_table, slots,
                  positions=None, last_idx=None):
    """row_slots [B] int32 (< 0: padding row); cu [B+1] int32 or None (then every row has
    tokens_per_row tokens); outputs are int32 device tensors: starts/kv_lens [B], block_table
    [B, W] (contiguous rows), slots/positions [N], last_idx [B]."""
    B = row_slots.shape[0]
    for t in (row_slots, starts, kv_lens, block_table, slots, positions, last_idx, cu):
        assert t is None or (t.is_cuda and t.dtype == torch.int32), "int32 GPU tensors only"
    assert block_table.dim() == 2 and block_table.shape[0] == B and block_table.is_contiguous()
    tables, lens = cache.dev_tables, cache.dev_lens
    lib = _lib.load()
    ptr = lambda t: t.data_ptr() if t is not None else None  # noqa: E731
    _lib.check(lib.mi_fa2_step_metadata(
        ptr(row_slots), ptr(cu), int(tokens_per_row), B, lens.data_ptr(), tables.shape[0],
        tables.data_ptr(), tables.stride(0), cache.block_size, block_table.shape[1],
        starts.data_ptr(), kv_lens.data_ptr(), block_table.data_ptr(), slots.data_ptr(),
        ptr(positions), ptr(last_idx), _lib.stream_of(row_slots)))

"""Paged KV cache feeding the MI355X paged attention kernels.

Same layout and bookkeeping as the reference's KVCache (kv_cache.py:8-121): one buffer
[num_layers, 2, num_blocks * block_size, num_kv_heads, head_dim] (dim 1: k=0, v=1), a free list of
blocks, per-sequence block tables, and logical token p of a sequence at physical slot
table[p // block_size] * block_size + p % block_size (kv_cache.py:15-16).  The API (alloc, free,
length, blocks_needed, ensure_capacity, trim, prepare, advance, write, read) keeps the reference's
names and meaning.

What changes is the per-step metadata.  The reference builds a Python list per new token and a
dense [B, S] gather index every step (kv_cache.py:74-101), then copies every cached token of every
row into a dense tensor per layer (kv_cache.py:117-121).  Here prepare() builds, with vectorised
numpy and ONE pinned host-to-device copy, exactly what the paged kernel reads:

  * block_table [B, W] int32 (rows padded with block 0, kv_cache.py:95),
  * kv_lens [B] int32 (keys per row after this step, model.py:175),
  * slot_mapping [B*T] (where this step's new tokens go, for write()),

and no per-layer gather happens on the GPU path.  read() (the dense gather) is kept for the CPU
fallback and for reference-compatible callers.

On the GPU the tables themselves are device-resident (device_tables, the default there): every
sequence holds a slot with a row of `dev_tables` [max_seqs, max_blocks_per_seq] int32 and a
length in `dev_lens` [max_seqs] int32 (both bounded independently of the pool size, so the tables
stay small for a pool of any size: 4096 x 2048 x 4 B = 32 MB at most by default).  A table row is written only when blocks are allocated
(ensure_capacity: one small copy per allocation), and a step sends only its rows' slots: one HIP
launch (kernels.meta.step_metadata, csrc/step_meta.hip) derives starts, kv_lens, the batch block
table, every new token's slot (and positions / last indices for mixed steps) and advances the
device lengths in place.  The host keeps the same tables and lengths for scheduling decisions.

prepare_packed() builds the metadata of a mixed step, where each row appends its own number of
tokens (one for a decoding chat, a whole prompt for a newly admitted one) and the rows' tokens are
packed back to back: prefix offsets cu_q, every token's position and slot, and each row's last
token (whose logits are sampled).
"""
import math
from dataclasses import dataclass, field

import numpy as np
import torch


@dataclass
class StepMeta:
    """Metadata of one forward step over rows `seqs`, each appending T tokens."""
    starts: list                 # tokens each row held before this step (host ints)
    T: int
    block_size: int
    starts_dev: torch.Tensor     # [B] int32
    kv_lens: torch.Tensor        # [B] int32 = starts + T
    slot_mapping: torch.Tensor   # [B*T] int64, row-major (row, t)
    block_table: torch.Tensor    # [B, W] int32
    slot_mapping32: torch.Tensor = None  # the same slots as int32 (for the fused RoPE + write)
    tables: list = field(default_factory=list)  # host copies of the rows' block lists
    kv_cap: int = None           # fixed upper bound of kv_lens (captured decode graphs)
    packed = False

    @property
    def max_kv(self):
        return self.kv_cap if self.kv_cap is not None else max(self.starts) + self.T

    def gather_idx(self, device):
        """[B, S] physical slot of every logical position [0, max_kv) (kv_cache.py:93-98)."""
        S, bs = self.max_kv, self.block_size
        pos = torch.arange(S, device=device)
        bt = self.block_table.to(device).long()
        return bt[:, pos // bs] * bs + pos % bs


@dataclass
class PackedMeta:
    """Metadata of one mixed step: row b appends counts[b] >= 1 tokens, packed back to back in row
    order (row b's tokens are [cu_q[b], cu_q[b+1]) of the packed batch)."""
    starts: list                 # tokens each row held before this step (host ints)
    counts: list                 # new tokens per row (host ints)
    block_size: int
    n_single: int                # leading rows with exactly one new token (decode-shaped rows)
    cu_q: torch.Tensor           # [B+1] int32
    kv_lens: torch.Tensor        # [B] int32 = starts + counts
    positions: torch.Tensor      # [N] int32: position of each packed token in its row
    slot_mapping32: torch.Tensor  # [N] int32: cache slot of each packed token
    last_idx: torch.Tensor       # [B] int32: packed index of each row's last token
    block_table: torch.Tensor    # [B, W] int32
    tables: list = field(default_factory=list)
    packed = True

    def split(self):
        """(max kv_len of the leading one-token rows, of the other rows, max new tokens of the
        other rows): the host bounds each attention launch is sized by."""
        D = self.n_single
        kv = [s + c for s, c in zip(self.starts, self.counts)]
        return (max(kv[:D], default=0), max(kv[D:], default=0), max(self.counts[D:], default=0))

    @property
    def max_kv(self):
        return max(s + c for s, c in zip(self.starts, self.counts))

    @property
    def max_q(self):
        return max(self.counts)

    @property
    def slot_mapping(self):
        return self.slot_mapping32.long()


class KVCache:
    # Default cap of one sequence's length: Qwen2.5's context window.
    DEFAULT_MAX_TOKENS_PER_SEQ = 32768
    DEFAULT_MAX_SEQS = 4096

    def __init__(self, num_blocks, block_size, device, dtype, num_layers, num_kv_heads, head_dim,
                 *, device_tables=None, max_seqs=None, max_blocks_per_seq=None):
        self.buf = torch.zeros(num_layers, 2, num_blocks * block_size, num_kv_heads, head_dim,
                               device=device, dtype=dtype)
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.device = torch.device(device)
        self._free_blocks = list(range(num_blocks))
        self._block_tables = {}   # seq id -> list of block ids, in logical order
        self._lengths = {}        # seq id -> tokens written so far
        self._next_seq = 0
        self.device_tables = self.device.type == "cuda" if device_tables is None else device_tables
        # Blocks one sequence may hold.  With device tables this is the width of a table row: the
        # pool, capped at the default context length, so the tables do not grow with the square
        # of the pool.  Host tables limit nothing, so there (as in the reference's KVCache) a
        # sequence may hold the whole pool unless the caller sets a cap.
        if max_blocks_per_seq is None:
            max_blocks_per_seq = (math.ceil(self.DEFAULT_MAX_TOKENS_PER_SEQ / block_size)
                                  if self.device_tables else num_blocks)
        self.max_blocks_per_seq = max(1, min(num_blocks, max_blocks_per_seq))
        # Sequence slots (rows of the device tables).  Every sequence that holds cache holds at
        # least one block once its first token is written, so num_blocks + a few transient empty
        # sequences bound how many can be live; the default takes that bound up to 4096 slots (the
        # scheduler evicts idle conversations when slots run out).
        if max_seqs is None:
            max_seqs = min(num_blocks + 16, self.DEFAULT_MAX_SEQS)
        self.max_seqs = max_seqs
        self._free_slots = list(range(self.max_seqs - 1, -1, -1))
        self.slot = {}            # seq id -> slot
        if self.device_tables:
            assert self.device.type == "cuda", "device-resident tables need a GPU cache"
            self.dev_tables = torch.zeros(self.max_seqs, self.max_blocks_per_seq, dtype=torch.int32,
                                          device=device)
            self.dev_lens = torch.zeros(self.max_seqs, dtype=torch.int32, device=device)

    # -- bookkeeping (kv_cache.py:31-72) -------------------------------------------------------
    def free_block_count(self):
        return len(self._free_blocks)

    def free_slot_count(self):
        return len(self._free_slots)

    def blocks_needed(self, seq, total_len):
        held = len(self._block_tables[seq]) if seq is not None else 0
        return max(0, math.ceil(total_len / self.block_size) - held)

    def alloc(self):
        if not self._free_slots:
            raise RuntimeError(f"all {self.max_seqs} sequence slots are in use")
        slot = self._free_slots.pop()
        seq = self._next_seq
        self._next_seq += 1
        self._block_tables[seq] = []
        self._lengths[seq] = 0
        self.slot[seq] = slot
        if self.device_tables:
            self.dev_lens[slot:slot + 1].zero_()
        return seq

    def free(self, seq):
        self._free_blocks.extend(self._block_tables.pop(seq))
        del self._lengths[seq]
        self._free_slots.append(self.slot.pop(seq))

    def length(self, seq):
        return self._lengths[seq]

    def ensure_capacity(self, seq, total_len):
        need = self.blocks_needed(seq, total_len)
        if need > len(self._free_blocks):
            raise RuntimeError(f"KV cache exhausted: seq {seq} needs {need} more blocks, "
                               f"only {len(self._free_blocks)} free")
        if len(self._block_tables[seq]) + need > self.max_blocks_per_seq:
            raise RuntimeError(f"seq {seq} would hold {len(self._block_tables[seq]) + need} blocks; "
                               f"a sequence holds at most {self.max_blocks_per_seq}")
        table = self._block_tables[seq]
        old = len(table)
        for _ in range(need):
            table.append(self._free_blocks.pop())
        if self.device_tables and need:
            new = torch.tensor(table[old:], dtype=torch.int32)
            self.dev_tables[self.slot[seq], old:old + need].copy_(new)

    def trim(self, seq):
        table = self._block_tables[seq]
        keep = math.ceil(self._lengths[seq] / self.block_size)
        self._free_blocks.extend(table[keep:])
        del table[keep:]

    def advance(self, seqs, T):
        """Count T new tokens (an int, or one count per row) as written."""
        counts = T if isinstance(T, (list, tuple)) else [T] * len(seqs)
        for s, c in zip(seqs, counts):
            self._lengths[s] += c

    # -- per-step metadata ----------------------------------------------------------------------
    def pack_step(self, seqs, T, W=None, out=None, rows=None):
        """Grow the rows' tables for T new tokens and pack the step's metadata into one int32 host
        array [starts | kv_lens | block_table rows*W | slot_mapping rows*T] (kv_cache.py:74-101).

        W defaults to the blocks the longest row needs; `rows` >= len(seqs) pads the batch with
        empty rows (no keys, slot -1: nothing read or written).  Returns (array, starts, W)."""
        bs = self.block_size
        starts = [self._lengths[s] for s in seqs]
        for s, start in zip(seqs, starts):
            self.ensure_capacity(s, start + T)
        B = len(seqs)
        R = rows or B
        W = W or max(1, math.ceil((max(starts) + T) / bs))
        tables = [self._block_tables[s] for s in seqs]
        n_all = 2 * R + R * W + R * T
        host = np.zeros(n_all, dtype=np.int32) if out is None else out[:n_all]
        if out is not None:
            host.fill(0)
        st = np.asarray(starts, dtype=np.int32)
        host[:B] = st
        host[R:R + B] = st + T
        bt = host[2 * R:2 * R + R * W].reshape(R, W)
        for i, t in enumerate(tables):
            n = min(len(t), W)
            bt[i, :n] = t[:n]
        pos = st[:, None] + np.arange(T, dtype=np.int32)[None, :]        # [B, T]
        sm = host[2 * R + R * W:].reshape(R, T)
        sm[:B] = bt[np.arange(B)[:, None], pos // bs] * bs + pos % bs
        sm[B:] = -1
        return host, starts, W

    def prepare(self, seqs, T):
        if self.device_tables:
            return self._prepare_device(seqs, [T] * len(seqs), packed=False)
        B = len(seqs)
        host, starts, W = self.pack_step(seqs, T)
        tables = [self._block_tables[s] for s in seqs]
        cpu = torch.from_numpy(host)
        if self.device.type == "cuda":
            dev = cpu.pin_memory().to(self.device, non_blocking=True)
        else:
            dev = cpu.clone()
        return StepMeta(
            starts=starts, T=T, block_size=self.block_size,
            starts_dev=dev[:B], kv_lens=dev[B:2 * B],
            block_table=dev[2 * B:2 * B + B * W].view(B, W),
            slot_mapping=dev[2 * B + B * W:].long(),
            slot_mapping32=dev[2 * B + B * W:],
            tables=[list(t) for t in tables])

    def prepare_packed(self, seqs, counts):
        """Grow the rows' tables for counts[b] new tokens each and build a PackedMeta with one
        pinned host-to-device copy of [cu_q | kv_lens | positions | slots | last_idx | tables]."""
        assert len(seqs) == len(counts) and len(seqs) > 0 and min(counts) >= 1
        if self.device_tables:
            return self._prepare_device(seqs, counts, packed=True)
        bs = self.block_size
        starts = [self._lengths[s] for s in seqs]
        for s, start, c in zip(seqs, starts, counts):
            self.ensure_capacity(s, start + c)
        B, N = len(seqs), sum(counts)
        st = np.asarray(starts, dtype=np.int32)
        cnt = np.asarray(counts, dtype=np.int32)
        kv = st + cnt
        W = max(1, math.ceil(int(kv.max()) / bs))
        tables = [self._block_tables[s] for s in seqs]
        host = np.zeros(2 * B + 1 + 2 * N + B + B * W, dtype=np.int32)
        cu = host[:B + 1]
        np.cumsum(cnt, out=cu[1:])
        host[B + 1:2 * B + 1] = kv
        o = 2 * B + 1
        row = np.repeat(np.arange(B), cnt)                          # row of each packed token
        pos = host[o:o + N]
        pos[:] = st[row] + (np.arange(N, dtype=np.int32) - cu[:-1][row])
        bt = host[o + 2 * N + B:].reshape(B, W)
        for i, t in enumerate(tables):
            n = min(len(t), W)
            bt[i, :n] = t[:n]
        host[o + N:o + 2 * N] = bt[row, pos // bs] * bs + pos % bs
        host[o + 2 * N:o + 2 * N + B] = cu[1:] - 1
        n_single = 0
        while n_single < B and counts[n_single] == 1:
            n_single += 1
        cpu = torch.from_numpy(host)
        if self.device.type == "cuda":
            dev = cpu.pin_memory().to(self.device, non_blocking=True)
        else:
            dev = cpu.clone()
        return PackedMeta(
            starts=starts, counts=list(counts), block_size=bs, n_single=n_single,
            cu_q=dev[:B + 1], kv_lens=dev[B + 1:2 * B + 1], positions=dev[o:o + N],
            slot_mapping32=dev[o + N:o + 2 * N], last_idx=dev[o + 2 * N:o + 2 * N + B],
            block_table=dev[o + 2 * N + B:].view(B, W), tables=[list(t) for t in tables])

    def _prepare_device(self, seqs, counts, packed):
        """The device-table path of prepare / prepare_packed: one pinned copy of the rows' slots
        (and packed offsets), one metadata launch; tables and lengths never leave the device."""
        from kernels.meta import step_metadata
        assert len(set(seqs)) == len(seqs), "a sequence may appear once per step"
        bs = self.block_size
        starts = [self._lengths[s] for s in seqs]
        for s, start, c in zip(seqs, starts, counts):
            self.ensure_capacity(s, start + c)
        B, N = len(seqs), sum(counts)
        W = max(1, math.ceil(max(st + c for st, c in zip(starts, counts)) / bs))
        host = np.empty(B + (B + 1 if packed else 0), dtype=np.int32)
        host[:B] = [self.slot[s] for s in seqs]
        if packed:
            host[B] = 0
            np.cumsum(np.asarray(counts, dtype=np.int32), out=host[B + 1:])
        small = torch.from_numpy(host).pin_memory().to(self.device, non_blocking=True)
        row_slots, cu = small[:B], (small[B:] if packed else None)
        out = torch.empty(3 * B + B * W + 2 * N, dtype=torch.int32, device=self.device)
        o_starts, o_kv, o_last = out[:B], out[B:2 * B], out[2 * B:3 * B]
        o_bt = out[3 * B:3 * B + B * W].view(B, W)
        o_slots, o_pos = out[3 * B + B * W:3 * B + B * W + N], out[3 * B + B * W + N:]
        step_metadata(self, row_slots, cu, counts[0], o_starts, o_kv, o_bt, o_slots,
                      o_pos if packed else None, o_last if packed else None)
        tables = [list(self._block_tables[s]) for s in seqs]
        if not packed:
            return StepMeta(starts=starts, T=counts[0], block_size=bs, starts_dev=o_starts,
                            kv_lens=o_kv, slot_mapping=None, block_table=o_bt,
                            slot_mapping32=o_slots, tables=tables)
        n_single = 0
        while n_single < B and counts[n_single] == 1:
            n_single += 1
        return PackedMeta(starts=starts, counts=list(counts), block_size=bs, n_single=n_single,
                          cu_q=cu, kv_lens=o_kv, positions=o_pos, slot_mapping32=o_slots,
                          last_idx=o_last, block_table=o_bt, tables=tables)

    # -- data movement --------------------------------------------------------------------------
    def k_pool(self, layer):
        return self.buf[layer, 0]

    def v_pool(self, layer):
        return self.buf[layer, 1]

    def write(self, layer, meta, k, v):
        """Scatter this step's k/v [B, Hkv, T, d] into their slots (kv_cache.py:108-115)."""
        B, H, T, D = k.shape
        sm = meta.slot_mapping if meta.slot_mapping is not None else meta.slot_mapping32.long()
        self.buf[layer, 0].index_copy_(0, sm, k.transpose(1, 2).reshape(B * T, H, D))
        self.buf[layer, 1].index_copy_(0, sm, v.transpose(1, 2).reshape(B * T, H, D))

    def read_row(self, layer, table, n):
        """Dense [Hkv, n, d] copies of the first n keys/values of the sequence whose block list is
        `table`: one row of read()."""
        pos = torch.arange(n, device=self.buf.device)
        idx = torch.tensor(table, device=self.buf.device, dtype=torch.long)[pos // self.block_size]
        idx = idx * self.block_size + pos % self.block_size
        return self.buf[layer, 0][idx].transpose(0, 1), self.buf[layer, 1][idx].transpose(0, 1)

    def read(self, layer, meta):
        """Dense [B, Hkv, S, d] copies of every row's keys/values (kv_cache.py:117-121)."""
        idx = meta.gather_idx(self.buf.device)
        return (self.buf[layer, 0][idx].transpose(1, 2), self.buf[layer, 1][idx].transpose(1, 2))

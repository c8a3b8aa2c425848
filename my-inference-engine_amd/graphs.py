"""Captured decode steps: one HIP graph per batch bucket, replayed over static metadata buffers.

The reference launches every kernel of every decode step from Python (chat.py:257-308 drives
model.py:157-207 once per step); at 16 chats that launch overhead, not the GPU, sets the time per
output token.  This module captures the whole decode forward (28 layers: norms, projections,
fused RoPE + cache write, paged attention, MLP, final norm, logits) once per batch bucket
(1, 2, 4, 8, 16 rows by default) and replays it.  Sampling stays outside the graph.

What varies from step to step lives in device buffers the graph reads.  With the cache's
device-resident tables (the default on the GPU) that is only [row slots | token ids], one small
host-to-device copy per step: the graph itself starts with the metadata launch
(kernels.meta.step_metadata), which reads the rows' tables and lengths on the device, writes
starts, kv_lens, the batch block table and the new tokens' cache slots, and advances the lengths.
Without device tables the graph reads a host-packed [starts | kv_lens | block_table rows x W |
slot_mapping rows] buffer (KVCache.pack_step's layout) and the token ids, two copies per step.
Either way W = the most blocks one sequence may hold, so any sequence fits and the attention
kernel's grid and workspace (sized for W*block_size keys) never change: its work split follows the
actual kv_lens on the device.  A batch smaller than its bucket is padded with empty rows (slot -1: no keys,
nothing written to the cache, zeros from attention), whose logits are ignored.
"""
import numpy as np
import torch

from kernels.meta import step_metadata
from kv_cache import StepMeta


class DecodeGraphs:
    def __init__(self, model, cache, buckets=(1, 2, 4, 8, 16)):
        assert cache.device.type == "cuda", "decode graphs need the GPU"
        self.model = model
        self.cache = cache
        self.W = cache.max_blocks_per_seq
        self.buckets = sorted(buckets)
        self.graphs = {}
        # One capture stream for all buckets, alive as long as the graphs: the kernels' workspace
        # is kept per stream, and a stream handle recycled by torch's pool while these graphs
        # exist would hand their workspace to unrelated calls.
        self._side = torch.cuda.Stream(device=cache.device)
        for rows in self.buckets:
            self._capture(rows)

    @property
    def max_rows(self):
        return self.buckets[-1]

    def _bucket(self, n):
        for b in self.buckets:
            if b >= n:
                return b
        raise ValueError(f"batch of {n} rows is larger than the largest captured bucket")

    def _capture(self, rows):
        dev, W, bs = self.cache.device, self.W, self.cache.block_size
        cache = self.cache
        if cache.device_tables:
            inp = torch.zeros(2 * rows, dtype=torch.int32, device=dev)   # [row slots | ids]
            inp[:rows] = -1                  # padding rows: nothing advances while warming up
            row_slots, ids_dev = inp[:rows], inp[rows:].view(rows, 1)
            out = torch.zeros(2 * rows + rows * W + rows, dtype=torch.int32, device=dev)
            meta = StepMeta(starts=None, T=1, block_size=bs, starts_dev=out[:rows],
                            kv_lens=out[rows:2 * rows],
                            block_table=out[2 * rows:2 * rows + rows * W].view(rows, W),
                            slot_mapping=None, slot_mapping32=out[2 * rows + rows * W:],
                            kv_cap=W * bs)

            def step():
                step_metadata(cache, row_slots, None, 1, meta.starts_dev, meta.kv_lens,
                              meta.block_table, meta.slot_mapping32)
                return self.model.forward_meta(ids_dev, cache, meta)
            host = torch.zeros(2 * rows, dtype=torch.int32).pin_memory()
            # `out` is written by every replay: it lives as long as the graph (it was allocated
            # before the capture, so the graph's own memory pool does not hold it)
            bufs = (inp, host, out)
        else:
            n_meta = 2 * rows + rows * W + rows
            meta_dev = torch.zeros(n_meta, dtype=torch.int32, device=dev)
            meta_dev[2 * rows + rows * W:] = -1      # no slot: nothing is written while warming up
            ids_dev = torch.zeros(rows, 1, dtype=torch.long, device=dev)
            meta = StepMeta(starts=None, T=1, block_size=bs, starts_dev=meta_dev[:rows],
                            kv_lens=meta_dev[rows:2 * rows],
                            block_table=meta_dev[2 * rows:2 * rows + rows * W].view(rows, W),
                            slot_mapping=None, slot_mapping32=meta_dev[2 * rows + rows * W:],
                            kv_cap=W * bs)

            def step():
                return self.model.forward_meta(ids_dev, cache, meta)
            bufs = (meta_dev, ids_dev, torch.zeros(n_meta, dtype=torch.int32).pin_memory(),
                    torch.zeros(rows, 1, dtype=torch.long).pin_memory())
        side = self._side
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(2):                       # allocations and workspaces happen here
                step()
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph), torch.no_grad():
            logits = step()
        self.graphs[rows] = (graph, logits, bufs, torch.cuda.Event())

    def run(self, seqs, tokens):
        """One decode step for cache sequences `seqs` fed `tokens` (one id per row); returns the
        rows' logits [len(seqs), vocab] (a view of the graph's output buffer, valid until the next
        replay of the same bucket)."""
        n = len(seqs)
        rows = self._bucket(n)
        graph, logits, bufs, copied = self.graphs[rows]
        copied.synchronize()             # the previous upload from these host buffers is done
        cache = self.cache
        if cache.device_tables:
            assert len(set(seqs)) == n, "a sequence may appear once per step"
            inp, host, _ = bufs
            for s in seqs:
                cache.ensure_capacity(s, cache.length(s) + 1)
            h = host.numpy()
            h[:n] = [cache.slot[s] for s in seqs]
            h[n:rows] = -1
            h[rows:rows + n] = tokens
            h[rows + n:] = 0
            inp.copy_(host, non_blocking=True)
        else:
            meta_dev, ids_dev, host_meta, host_ids = bufs
            cache.pack_step(seqs, 1, W=self.W, out=host_meta.numpy(), rows=rows)
            ids = host_ids.numpy()
            ids[:n, 0] = tokens
            ids[n:, 0] = 0
            meta_dev.copy_(host_meta, non_blocking=True)
            ids_dev.copy_(host_ids, non_blocking=True)
        copied.record()
        graph.replay()
        cache.advance(seqs, 1)
        return logits[:n, -1]

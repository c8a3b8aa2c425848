"""Captured decode steps: one HIP graph per batch bucket, replayed over static metadata buffers.

The reference launches every kernel of every decode step from Python (chat.py:257-308 drives
model.py:157-207 once per step); at 16 chats that launch overhead, not the GPU, sets the time per
output token.  This module captures the whole decode forward (28 layers: norms, projections,
fused RoPE + cache write, paged attention, MLP, final norm, logits) once per batch bucket
(1, 2, 4, 8, 16 rows by default) and replays it.  Sampling stays outside the graph.

What varies from step to step lives in device buffers the graph reads:
  * the packed step metadata [starts | kv_lens | block_table rows x W | slot_mapping rows] (the
    same layout KVCache.prepare builds), with W = the pool's block count, so any sequence fits and
    the attention kernel's grid and workspace (sized for W*block_size keys) never change: its
    work split follows the actual kv_lens on the device;
  * the input token ids.
Both are refreshed by one host-to-device copy each before a replay.  A batch smaller than its
bucket is padded with empty rows (no keys, cache slot -1: the fused cache write skips them, the
attention kernel returns zeros for them), whose logits are ignored.
"""
import numpy as np
import torch

from kv_cache import StepMeta


class DecodeGraphs:
    def __init__(self, model, cache, buckets=(1, 2, 4, 8, 16)):
        assert cache.device.type == "cuda", "decode graphs need the GPU"
        self.model = model
        self.cache = cache
        self.W = cache.num_blocks
        self.buckets = sorted(buckets)
        self.graphs = {}
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
        n_meta = 2 * rows + rows * W + rows
        meta_dev = torch.zeros(n_meta, dtype=torch.int32, device=dev)
        meta_dev[2 * rows + rows * W:] = -1          # no slot: nothing is written while warming up
        ids_dev = torch.zeros(rows, 1, dtype=torch.long, device=dev)
        meta = StepMeta(starts=None, T=1, block_size=bs, starts_dev=meta_dev[:rows],
                        kv_lens=meta_dev[rows:2 * rows],
                        block_table=meta_dev[2 * rows:2 * rows + rows * W].view(rows, W),
                        slot_mapping=None, slot_mapping32=meta_dev[2 * rows + rows * W:],
                        kv_cap=W * bs)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(2):                       # allocations and workspaces happen here
                self.model.forward_meta(ids_dev, self.cache, meta)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph), torch.no_grad():
            logits = self.model.forward_meta(ids_dev, self.cache, meta)
        host_meta = torch.zeros(n_meta, dtype=torch.int32).pin_memory()
        host_ids = torch.zeros(rows, 1, dtype=torch.long).pin_memory()
        self.graphs[rows] = (graph, meta_dev, ids_dev, logits, host_meta, host_ids)

    def run(self, seqs, tokens):
        """One decode step for cache sequences `seqs` fed `tokens` (one id per row); returns the
        rows' logits [len(seqs), vocab] (a view of the graph's output buffer, valid until the next
        replay of the same bucket)."""
        n = len(seqs)
        rows = self._bucket(n)
        graph, meta_dev, ids_dev, logits, host_meta, host_ids = self.graphs[rows]
        self.cache.pack_step(seqs, 1, W=self.W, out=host_meta.numpy(), rows=rows)
        ids = host_ids.numpy()
        ids[:n, 0] = tokens
        ids[n:, 0] = 0
        meta_dev.copy_(host_meta, non_blocking=True)
        ids_dev.copy_(host_ids, non_blocking=True)
        graph.replay()
        self.cache.advance(seqs, 1)
        return logits[:n, -1]

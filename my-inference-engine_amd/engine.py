"""Continuous-batching scheduler over the paged KV cache (the caller of the attention path).

Restates the reference engine's scheduling semantics (chat.py) as one class instead of module
globals and a daemon worker thread:

  * a message is admitted only if its conversation's history + prompt + a full reply (+ the
    trailing separator) fit in free blocks (chat.py:117-125), evicting idle conversations
    least-recently-used first (chat.py:128-146); one that can never fit is rejected
    (chat.py:214-225), one that does not fit yet is deferred and retried every tick
    (chat.py:221-229,236-239);
  * admission runs one un-chunked prefill over the tokens the cache does not hold yet and samples
    the first reply token (chat.py:157-185); at most one admission per tick, so decoding jobs are
    not starved (chat.py:247-253);
  * every tick then runs ONE batched decode step for all active jobs (chat.py:257-308) and samples
    every row with a single device sync (chat.py:103-107); on the GPU the draw is one fused HIP
    launch (kernels.sample.sample_tokens: the exponential race torch.multinomial uses, over a
    Philox stream keyed by the engine's seed and advanced once per draw), on the CPU the
    reference's softmax + multinomial;
  * a finished reply keeps its cache (the conversation continues), appends the separator and
    gives back reserved-but-unused blocks (chat.py:194-211).

With mixed_prefill=True the admission rules stay, but an admitted prompt no longer runs a forward
of its own: its tokens join the tick's decode step as one more row of a packed mixed batch
(Qwen2ForCausalLM.forward_mixed), and its first reply token is sampled with the decode rows.  Then
several prompts may be admitted per tick, up to max_step_tokens prompt tokens (one prompt is always
admitted, however long, as the reference's un-chunked prefill is).

Tokenizer, stop sequences, streaming listeners and the web UI are outside the attention path and
not rebuilt; conversations carry token ids.
"""
import time
from collections import deque
from dataclasses import dataclass, field

import torch

from kernels.sample import sample_tokens


@dataclass
class Conversation:
    ids: list = field(default_factory=list)  # full token history
    seq: object = None                       # cache sequence id, None until admitted / after eviction
    eos_id: int = -1                         # -1: no token ends a reply (chat.py:323, NO_EOS)


@dataclass
class Job:
    conv: Conversation
    new_ids: list
    max_tokens: int
    next_token: int = None
    steps: int = 0
    generated: list = field(default_factory=list)
    t_submit: float = 0.0
    t_first: float = None
    t_done: float = None
    rejected: str = None
    prefill: list = None   # mixed mode: prompt tokens waiting for the next step


class Engine:
    def __init__(self, model, cache, *, max_reply_tokens=512, temperature=1.0, sep_ids=(198,),
                 seed=0, decode_graphs=None, mixed_prefill=False, max_step_tokens=16384):
        self.model = model
        self.mixed_prefill = mixed_prefill
        self.max_step_tokens = max_step_tokens
        self.cache = cache
        self.decode_graphs = decode_graphs  # graphs.DecodeGraphs, or None: eager decode steps
        self.max_reply_tokens = max_reply_tokens
        self.temperature = temperature
        self.sep_ids = list(sep_ids)   # appended after each reply, like "\n" (chat.py:200)
        self.device = next(model.parameters()).device
        self.seed = seed
        self.gen = torch.Generator(device=self.device).manual_seed(seed)
        self._draws = 0      # Philox offset of the fused sampler: one per sampling call
        self.queue = deque()
        self.active = []
        self.deferred = []
        self.resident = []   # conversations holding cache, least recently used first
        self.finished = []

    # -- public ---------------------------------------------------------------------------------
    def submit(self, conv, new_ids, max_tokens=None):
        job = Job(conv, list(new_ids), max_tokens or self.max_reply_tokens,
                  t_submit=time.perf_counter())
        self.queue.append(job)
        return job

    def release(self, conv):
        """Free a conversation's blocks now (chat.py:325-330)."""
        if conv.seq is not None:
            self._evict(conv)

    def idle(self):
        return not (self.queue or self.active or self.deferred)

    def tick(self):
        """One worker iteration (chat.py:232-254)."""
        if self.mixed_prefill:
            return self._tick_mixed()
        for job in list(self.deferred):
            if self._make_room(job):
                self.deferred.remove(job)
                self._admit(job)
        if not self.active and not self.deferred:
            if self.queue:  # the reference blocks on its queue here
                self._try_admit_or_defer(self.queue.popleft())
        elif not self.active:
            pass  # deferred jobs wait for blocks to be released (the reference sleeps)
        elif self.queue:
            self._try_admit_or_defer(self.queue.popleft())
        self._process()

    def _tick_mixed(self):
        """Admissions fill the step's prompt-token budget; deferred jobs go first, then the queue
        until a job has to wait.  With nothing active and jobs deferred, new ones wait too (the
        reference sleeps there)."""
        budget = [self.max_step_tokens]

        def fits(job):
            n = len(job.conv.ids) + len(job.new_ids) - (
                self.cache.length(job.conv.seq) if job.conv.seq is not None else 0)
            return n <= budget[0] or not any(j.prefill is not None for j in self.active)

        def admit(job):
            self._admit(job)
            budget[0] -= len(job.prefill)

        for job in list(self.deferred):
            if fits(job) and self._make_room(job):
                self.deferred.remove(job)
                admit(job)
        if self.active or not self.deferred:
            while self.queue and fits(self.queue[0]):
                job = self.queue.popleft()
                before = len(self.deferred)
                self._try_admit_or_defer(job)
                if job in self.active:
                    budget[0] -= len(job.prefill)
                elif len(self.deferred) > before:
                    break
        self._process()

    def run_until_idle(self, max_ticks=1_000_000, on_tick=None):
        """Tick until nothing is queued, deferred or active; on_tick() runs after every tick."""
        for _ in range(max_ticks):
            if self.idle():
                return
            if not self.active and self.deferred and not self.queue and not any(
                    self._fits_after_eviction(j) for j in self.deferred):
                raise RuntimeError("deferred jobs can never be admitted: nothing else will "
                                   "release cache blocks")
            self.tick()
            if on_tick is not None:
                on_tick()
        raise RuntimeError("scheduler did not drain")

    def _fits_after_eviction(self, job):
        idle_blocks = sum(len(self.cache._block_tables[c.seq]) for c in self.resident
                          if c.seq is not None and c is not job.conv)
        need = self.cache.blocks_needed(job.conv.seq, self._reserve_len(job))
        return need <= self.cache.free_block_count() + idle_blocks

    # -- scheduling -----------------------------------------------------------------------------
    def _reserve_len(self, job):
        return len(job.conv.ids) + len(job.new_ids) + job.max_tokens + len(self.sep_ids)

    def _evict(self, conv):
        self.cache.free(conv.seq)
        conv.seq = None
        if conv in self.resident:
            self.resident.remove(conv)

    def _make_room(self, job):
        """Evict idle conversations, least recently used first, until the job's reservation fits
        in free blocks (chat.py:128-146) and, for a conversation without cache, a sequence slot is
        free."""
        busy = {id(j.conv) for j in self.active} | {id(job.conv)}

        def short():
            return (self.cache.blocks_needed(job.conv.seq, self._reserve_len(job))
                    > self.cache.free_block_count()
                    or (job.conv.seq is None and self.cache.free_slot_count() == 0))
        while short():
            idle = [c for c in self.resident if id(c) not in busy]
            if not idle:
                return False
            self._evict(idle[0])
        return True

    def _touch(self, conv):
        if conv in self.resident:
            self.resident.remove(conv)
        self.resident.append(conv)

    def _try_admit_or_defer(self, job):
        if self.cache.blocks_needed(None, self._reserve_len(job)) > min(
                self.cache.num_blocks, self.cache.max_blocks_per_seq):
            job.rejected = "conversation is too long for the KV cache"
            job.t_done = time.perf_counter()
            self.finished.append(job)
        elif self._make_room(job):
            self._admit(job)
        else:
            self.deferred.append(job)

    def _admit(self, job):
        conv = job.conv
        reserve = self._reserve_len(job)
        conv.ids.extend(job.new_ids)
        if conv.seq is None:
            conv.seq = self.cache.alloc()
        prefill = conv.ids[self.cache.length(conv.seq):]
        self.cache.ensure_capacity(conv.seq, reserve)
        self._touch(conv)
        if self.mixed_prefill:
            job.prefill = prefill     # runs inside the next step, as one more row
            self.active.append(job)
            return
        input_ids = torch.tensor([prefill], device=self.device)
        with torch.no_grad():
            logits = self.model(input_ids, self.cache, [conv.seq])
        job.next_token = self._sample(logits[:, -1])[0]
        job.t_first = time.perf_counter()
        self.active.append(job)

    def _finish(self, job):
        conv = job.conv
        conv.ids.extend(self.sep_ids)
        self.cache.trim(conv.seq)
        self._touch(conv)
        job.t_done = time.perf_counter()
        self.active.remove(job)
        self.finished.append(job)

    def _process(self):
        continuing, prompts = [], []
        for job in list(self.active):
            if job.prefill is not None:
                prompts.append(job)
                continue
            tok = job.next_token
            job.conv.ids.append(tok)
            job.generated.append(tok)
            if tok == job.conv.eos_id:
                self._finish(job)
                continue
            job.steps += 1
            if job.steps >= job.max_tokens:
                self._finish(job)
                continue
            continuing.append(job)
        if prompts:
            return self._step_mixed(continuing, prompts)
        if not continuing:
            return
        seqs = [j.conv.seq for j in continuing]
        graphs = self.decode_graphs
        if graphs is not None and len(seqs) <= graphs.max_rows:
            last = graphs.run(seqs, [j.next_token for j in continuing])
        else:
            input_ids = torch.tensor([[j.next_token] for j in continuing], device=self.device)
            with torch.no_grad():
                last = self.model(input_ids, self.cache, seqs)[:, -1]
        for job, tok in zip(continuing, self._sample(last)):
            job.next_token = tok

    def _step_mixed(self, continuing, prompts):
        """One packed step: the decode rows first (one token each), then the admitted prompts."""
        jobs = continuing + prompts
        rows = [[j.next_token] for j in continuing] + [j.prefill for j in prompts]
        with torch.no_grad():
            logits = self.model.forward_mixed(rows, self.cache, [j.conv.seq for j in jobs])
        toks = self._sample(logits)
        now = time.perf_counter()
        for job, tok in zip(jobs, toks):
            job.next_token = tok
        for job in prompts:
            job.prefill = None
            job.t_first = now

    def _sample(self, logits):
        """One id per row of [B, vocab] logits, one device sync for all rows (chat.py:103-107)."""
        if logits.is_cuda:
            toks = sample_tokens(logits, self.temperature, self.seed, self._draws).tolist()
            self._draws += 1
            if min(toks) < 0:
                raise RuntimeError("a row of logits has no finite entry to sample from")
            return toks
        probs = torch.softmax(logits.float() / self.temperature, dim=-1)
        return torch.multinomial(probs, 1, generator=self.gen).squeeze(1).tolist()


def run_concurrent_chats(engine, prompts, reply_tokens):
    """Start len(prompts) fresh conversations at once and run them to completion.

    Returns the reference benchmark's summary (metrics/benchmark_concurrency.py:57-76): generated
    tokens / wall time from the first submit to the last finish, TTFT / latency percentiles,
    time per output token, the peak number of active (decoding) chats and the KV utilisation:
    the peak token count held by the chats' conversations as a percentage of the cache's token
    capacity (metrics/benchmark_concurrency.py:151-159,176, where the reference samples both
    from a thread every few milliseconds; here they are sampled after every scheduler tick, from
    host-side state only)."""
    convs = [Conversation() for _ in prompts]
    peak = {"active": 0, "cached": 0}

    def sample():
        peak["active"] = max(peak["active"], len(engine.active))
        peak["cached"] = max(peak["cached"], sum(len(c.ids) for c in convs if c.seq is not None))

    start = time.perf_counter()
    jobs = [engine.submit(c, p, reply_tokens) for c, p in zip(convs, prompts)]
    engine.run_until_idle(on_tick=sample)
    torch.cuda.synchronize() if engine.device.type == "cuda" else None
    wall = time.perf_counter() - start
    for c in convs:
        engine.release(c)

    def pct(vals, q):
        vals = sorted(vals)
        pos = q / 100 * (len(vals) - 1)
        lo, hi = int(pos), min(int(pos) + 1, len(vals) - 1)
        return vals[lo] + (vals[hi] - vals[lo]) * (pos - lo)

    tokens = sum(len(j.generated) for j in jobs)
    ttft = [j.t_first - j.t_submit for j in jobs]
    lat = [j.t_done - j.t_submit for j in jobs]
    tpot = [(j.t_done - j.t_first) / (len(j.generated) - 1) for j in jobs if len(j.generated) > 1]
    capacity = engine.cache.num_blocks * engine.cache.block_size
    return {"chats": len(prompts), "tokens": tokens, "wall_s": wall, "tok_per_s": tokens / wall,
            "ttft_p50": pct(ttft, 50), "ttft_p99": pct(ttft, 99), "lat_p50": pct(lat, 50),
            "lat_p99": pct(lat, 99), "tpot": sum(tpot) / max(1, len(tpot)),
            "peak_active": peak["active"], "kv_util": 100.0 * peak["cached"] / capacity}

"""CPU tests of the attention path's callers: the paged KV cache metadata, the Qwen2 model's use of
it, and the continuous-batching scheduler (chat.py semantics), forced into admission, deferral,
eviction and rejection with tiny block pools.  The model runs its CPU fallback (fp32 SDPA) here;
the GPU run of the same model through the HIP kernels is tests/test_engine_gpu.py."""
import math

import pytest

import torch

from engine import Conversation, Engine, run_concurrent_chats
from kv_cache import KVCache
from model import QwenConfig, Qwen2ForCausalLM
from oracle import paged as opaged

TINY = QwenConfig(hidden_size=256, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=128,
                  intermediate_size=512, vocab_size=300)


def tiny_model(seed=0):
    torch.manual_seed(seed)
    return Qwen2ForCausalLM(TINY).float().init_random(std=0.05, seed=seed).eval()


def tiny_cache(num_blocks=64, block_size=16):
    return KVCache(num_blocks, block_size, "cpu", torch.float32, TINY.num_layers, TINY.num_kv_heads,
                   TINY.head_dim)


def test_prepare_metadata_matches_slot_arithmetic():
    cache = tiny_cache(num_blocks=40)
    seqs = [cache.alloc() for _ in range(3)]
    cache.ensure_capacity(seqs[0], 37)
    cache._lengths[seqs[0]] = 37
    cache.ensure_capacity(seqs[2], 5)
    cache._lengths[seqs[2]] = 5
    meta = cache.prepare(seqs, 3)
    assert meta.starts == [37, 0, 5]
    assert meta.kv_lens.tolist() == [40, 3, 8]
    W = meta.block_table.shape[1]
    assert W == math.ceil(40 / 16)
    for b, s in enumerate(seqs):
        table = cache._block_tables[s]
        assert meta.block_table[b, :len(table)].tolist() == table[:W]
        for t in range(3):
            p = meta.starts[b] + t
            assert meta.slot_mapping[b * 3 + t].item() == opaged.slot_of(table, p, 16)


def test_cached_decode_equals_full_recompute():
    model = tiny_model()
    ids = torch.randint(0, TINY.vocab_size, (1, 23), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        c1 = tiny_cache()
        s1 = c1.alloc()
        model(ids[:, :20], c1, [s1])
        model(ids[:, 20:21], c1, [s1])
        model(ids[:, 21:22], c1, [s1])
        inc = model(ids[:, 22:23], c1, [s1])
        c2 = tiny_cache()
        s2 = c2.alloc()
        full = model(ids, c2, [s2])
    assert torch.allclose(inc, full, atol=1e-5, rtol=1e-4)


def test_ragged_batched_decode_equals_per_row_decode():
    model = tiny_model(1)
    g = torch.Generator().manual_seed(2)
    prompts = [torch.randint(0, TINY.vocab_size, (1, n), generator=g) for n in (5, 33, 17)]
    nxt = torch.randint(0, TINY.vocab_size, (3, 1), generator=g)
    with torch.no_grad():
        cache = tiny_cache()
        seqs = [cache.alloc() for _ in prompts]
        for s, p in zip(seqs, prompts):
            model(p, cache, [s])
        batched = model(nxt, cache, seqs)
        singles = []
        for i, p in enumerate(prompts):
            c = tiny_cache()
            s = c.alloc()
            model(p, c, [s])
            singles.append(model(nxt[i:i + 1], c, [s]))
    assert torch.allclose(batched, torch.cat(singles), atol=1e-5, rtol=1e-4)


def _engine(num_blocks, reply=4):
    return Engine(tiny_model(), tiny_cache(num_blocks=num_blocks), max_reply_tokens=reply, seed=0)


def test_every_job_generates_its_reply_and_blocks_come_back():
    eng = _engine(64)
    g = torch.Generator().manual_seed(3)
    prompts = [torch.randint(0, TINY.vocab_size, (n,), generator=g).tolist() for n in (7, 40, 3, 21)]
    summary = run_concurrent_chats(eng, prompts, reply_tokens=4)
    assert summary["tokens"] == 16
    assert all(len(j.generated) == 4 for j in eng.finished)
    assert eng.cache.free_block_count() == 64


def test_reservation_defers_until_blocks_free_up():
    # 6 blocks of 16 = 96 tokens; each job reserves 40 + 4 + 1 tokens = 3 blocks: two fit at once
    eng = _engine(6)
    convs = [Conversation() for _ in range(3)]
    jobs = [eng.submit(c, list(range(40)), 4) for c in convs]
    eng.tick()
    eng.tick()
    eng.tick()
    assert len(eng.active) + len(eng.finished) == 2 and not eng.queue and len(eng.deferred) == 1
    # finishing the first replies releases nothing (idle conversations keep their cache) until
    # eviction makes room: the deferred job is admitted by evicting the least recently used chat
    eng.run_until_idle()
    assert all(len(j.generated) == 4 for j in jobs)
    assert sum(c.seq is None for c in convs) >= 1


def test_impossible_conversation_is_rejected():
    eng = _engine(2)  # 32 tokens of cache
    job = eng.submit(Conversation(), list(range(40)), 4)
    eng.tick()
    assert job.rejected and job in eng.finished
    assert eng.cache.free_block_count() == 2


def test_eviction_is_least_recently_used_and_history_is_reprefilled():
    eng = _engine(8)
    a, b = Conversation(), Conversation()
    eng.submit(a, list(range(30)), 2)
    eng.run_until_idle()
    eng.submit(b, list(range(30)), 2)
    eng.run_until_idle()
    assert a.seq is not None and b.seq is not None
    # each idle chat holds 31 tokens = 2 blocks, 4 blocks are free; a third message of 80 tokens
    # reserves 80 + 2 + 1 tokens = 6 blocks: a (least recently used) is evicted, b is kept
    c = Conversation()
    eng.submit(c, list(range(80)), 2)
    eng.run_until_idle()
    assert a.seq is None and b.seq is not None
    # a's next turn re-prefills its whole history from a.ids
    n_hist = len(a.ids)
    job = eng.submit(a, [5, 6], 2)
    eng.run_until_idle()
    assert len(job.generated) == 2
    assert eng.cache.length(a.seq) == n_hist + 2 + 1  # history + new + first sampled token fed


def test_trim_returns_unused_reserved_blocks():
    eng = _engine(16, reply=40)
    conv = Conversation(eos_id=None)
    job = eng.submit(conv, list(range(10)), 40)
    conv.eos_id = None
    eng.tick()  # admitted: reserved 10 + 40 + 1 tokens = 4 blocks
    assert len(eng.cache._block_tables[conv.seq]) == 4
    job.max_tokens = 2  # end early
    eng.run_until_idle()
    assert len(eng.cache._block_tables[conv.seq]) == math.ceil(eng.cache.length(conv.seq) / 16)


# -- mixed prefill + decode steps ----------------------------------------------------------------

def test_prepare_packed_metadata_matches_slot_arithmetic():
    cache = tiny_cache(num_blocks=40)
    seqs = [cache.alloc() for _ in range(4)]
    for s, n in zip(seqs, (37, 16, 0, 5)):
        cache.ensure_capacity(s, n)
        cache._lengths[s] = n
    counts = [1, 1, 20, 3]
    meta = cache.prepare_packed(seqs, counts)
    assert meta.n_single == 2 and meta.starts == [37, 16, 0, 5]
    assert meta.cu_q.tolist() == [0, 1, 2, 22, 25]
    assert meta.kv_lens.tolist() == [38, 17, 20, 8]
    assert meta.last_idx.tolist() == [0, 1, 21, 24]
    assert meta.split() == (38, 20, 20)
    pos, slots = meta.positions.tolist(), meta.slot_mapping32.tolist()
    i = 0
    for b, s in enumerate(seqs):
        table = cache._block_tables[s]
        assert meta.block_table[b, :len(table)].tolist() == table[:meta.block_table.shape[1]]
        for t in range(counts[b]):
            assert pos[i] == meta.starts[b] + t
            assert slots[i] == opaged.slot_of(table, pos[i], 16)
            i += 1
    assert i == 25


def test_mixed_step_equals_separate_forwards():
    """Decode rows and new prompts packed into one step give each row the logits of running it on
    its own, and each row's cache length grows by its own count."""
    model = tiny_model(2)
    g = torch.Generator().manual_seed(5)
    hist = [torch.randint(0, TINY.vocab_size, (n,), generator=g).tolist() for n in (9, 40, 17)]
    nxt = torch.randint(0, TINY.vocab_size, (3,), generator=g).tolist()
    new = [torch.randint(0, TINY.vocab_size, (n,), generator=g).tolist() for n in (30, 1, 12)]
    with torch.no_grad():
        mc = tiny_cache()
        mseqs = [mc.alloc() for _ in range(6)]
        for s, h in zip(mseqs, hist):
            model(torch.tensor([h]), mc, [s])
        # rows 0-2 decode one token, rows 3-5 are prompts (one of them a single token)
        got = model.forward_mixed([[t] for t in nxt] + new, mc, mseqs)
        want = []
        for rows in [h + [t] for h, t in zip(hist, nxt)] + new:
            c = tiny_cache()
            s = c.alloc()
            want.append(model(torch.tensor([rows]), c, [s])[:, -1])
    assert torch.allclose(got, torch.cat(want), atol=1e-5, rtol=1e-4)
    assert [mc.length(s) for s in mseqs] == [10, 41, 18, 30, 1, 12]


def _mixed_engine(num_blocks, reply=4, **kw):
    return Engine(tiny_model(), tiny_cache(num_blocks=num_blocks), max_reply_tokens=reply, seed=0,
                  mixed_prefill=True, **kw)


def test_mixed_engine_admits_every_prompt_into_one_step():
    eng = _mixed_engine(64)
    g = torch.Generator().manual_seed(3)
    prompts = [torch.randint(0, TINY.vocab_size, (n,), generator=g).tolist() for n in (7, 40, 3, 21)]
    jobs = [eng.submit(Conversation(), p, 4) for p in prompts]
    eng.tick()
    assert len(eng.active) == 4 and all(j.t_first is not None and j.prefill is None for j in jobs)
    eng.run_until_idle()
    assert all(len(j.generated) == 4 for j in jobs)
    for j in jobs:
        eng.release(j.conv)
    assert eng.cache.free_block_count() == 64


def test_mixed_engine_respects_the_step_token_budget():
    eng = _mixed_engine(64, max_step_tokens=50)
    jobs = [eng.submit(Conversation(), list(range(n)), 4) for n in (30, 30, 60, 10)]
    eng.tick()   # 30 fits, the second 30 would pass 50: one admission
    assert [j in eng.active for j in jobs] == [True, False, False, False]
    eng.tick()   # a step with decode rows only still has the whole budget: 30, then 60 waits
    assert [j in eng.active for j in jobs] == [True, True, False, False]
    eng.tick()   # 60 > 50 but it is the step's first prompt: admitted alone (un-chunked)
    assert [j in eng.active for j in jobs] == [True, True, True, False]
    eng.run_until_idle()
    assert all(len(j.generated) == 4 for j in jobs)


def test_mixed_engine_defers_and_evicts_like_the_reference():
    eng = _mixed_engine(6)
    convs = [Conversation() for _ in range(3)]
    jobs = [eng.submit(c, list(range(40)), 4) for c in convs]
    eng.tick()
    # each job reserves 3 of the 6 blocks: two admitted in the first step, the third deferred
    assert len(eng.active) == 2 and not eng.queue and len(eng.deferred) == 1
    eng.run_until_idle()
    assert all(len(j.generated) == 4 for j in jobs)
    assert sum(c.seq is None for c in convs) >= 1


def test_mixed_and_separate_prefill_generate_the_same_tokens():
    """Near-greedy sampling (temperature 1e-4) makes the sampled ids a function of the logits
    only, so the two schedules must produce the same replies."""
    g = torch.Generator().manual_seed(7)
    prompts = [torch.randint(0, TINY.vocab_size, (n,), generator=g).tolist() for n in (7, 40, 3, 21, 16)]
    replies = []
    for mixed in (False, True):
        eng = Engine(tiny_model(), tiny_cache(num_blocks=64), max_reply_tokens=6, seed=0,
                     temperature=1e-4, mixed_prefill=mixed)
        jobs = [eng.submit(Conversation(), p, 6) for p in prompts]
        eng.run_until_idle()
        replies.append([j.generated for j in jobs])
    assert replies[0] == replies[1]


def test_idle_conversations_are_evicted_when_sequence_slots_run_out():
    # 64 blocks but only 3 sequence slots: the fourth conversation takes the slot of the least
    # recently used idle one instead of failing
    cache = KVCache(64, 16, "cpu", torch.float32, TINY.num_layers, TINY.num_kv_heads, TINY.head_dim,
                    max_seqs=3)
    eng = Engine(tiny_model(), cache, max_reply_tokens=2, seed=0)
    convs = [Conversation() for _ in range(4)]
    for c in convs:
        eng.submit(c, list(range(10)), 2)
        eng.run_until_idle()
    assert convs[0].seq is None and all(c.seq is not None for c in convs[1:])
    assert cache.free_slot_count() == 0 and len(cache.slot) == 3
    job = eng.submit(convs[0], [1, 2], 2)        # re-admitted: evicts convs[1], re-prefills history
    eng.run_until_idle()
    assert len(job.generated) == 2 and convs[1].seq is None and convs[0].seq is not None


def test_table_width_and_slots_are_bounded_independently_of_the_pool():
    """A sequence holds at most max_blocks_per_seq blocks and the slot count is capped.  The
    default cap (32,768 tokens) exists only to bound device tables; host tables limit nothing, so
    there a sequence may hold the whole pool, as in the reference's KVCache."""
    big = KVCache(5000, 16, "cpu", torch.float32, 1, 1, 8)
    assert big.max_blocks_per_seq == 5000 and big.max_seqs == 4096
    small = KVCache(100, 16, "cpu", torch.float32, 1, 1, 8)
    assert small.max_blocks_per_seq == 100 and small.max_seqs == 116
    c = KVCache(100, 16, "cpu", torch.float32, 1, 1, 8, max_blocks_per_seq=4)
    s = c.alloc()
    c.ensure_capacity(s, 64)  # exactly 4 blocks
    with pytest.raises(RuntimeError, match="at most 4"):
        c.ensure_capacity(s, 65)
    assert len(c._block_tables[s]) == 4 and c.free_block_count() == 96


def test_long_sequence_on_a_large_host_table_pool_is_accepted():
    """Host tables (the CPU path, or device_tables=False) accept a sequence longer than the
    device-table default cap: only the pool running out of blocks refuses it
    (the reference's kv_cache.py:55-64)."""
    c = KVCache(3000, 16, "cpu", torch.float32, 1, 1, 8)
    s = c.alloc()
    c.ensure_capacity(s, 40000)  # 2,500 blocks: past 32,768 tokens, within the pool
    assert len(c._block_tables[s]) == 2500 and c.free_block_count() == 500
    with pytest.raises(RuntimeError, match="exhausted"):
        c.ensure_capacity(s, 3001 * 16)


def test_concurrency_summary_reports_peak_active_and_kv_utilisation():
    # metrics/benchmark_concurrency.py:57-76,151-159,176: the peak number of active chats and the
    # peak tokens held by the chats' conversations as a share of the cache's capacity
    eng = _mixed_engine(64)
    g = torch.Generator().manual_seed(3)
    lens = (7, 40, 3, 21)
    prompts = [torch.randint(0, TINY.vocab_size, (n,), generator=g).tolist() for n in lens]
    summary = run_concurrent_chats(eng, prompts, reply_tokens=4)
    assert summary["peak_active"] == 4  # every prompt joins the first mixed step
    held = sum(lens) + len(lens) * (4 + 1)  # prompts, 4-token replies and the separator
    assert summary["kv_util"] == pytest.approx(100.0 * held / (64 * 16))
    # one prompt per tick (the reference's schedule) keeps fewer chats active at once
    eng = _engine(64)
    summary = run_concurrent_chats(eng, prompts, reply_tokens=4)
    assert 1 <= summary["peak_active"] <= 4
    assert summary["kv_util"] == pytest.approx(100.0 * held / (64 * 16))

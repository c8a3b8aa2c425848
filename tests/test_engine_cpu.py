"""CPU tests of the attention path's callers: the paged KV cache metadata, the Qwen2 model's use of
it, and the continuous-batching scheduler (chat.py semantics), forced into admission, deferral,
eviction and rejection with tiny block pools.  The model runs its CPU fallback (fp32 SDPA) here;
the GPU run of the same model through the HIP kernels is tests/test_engine_gpu.py."""
import math

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

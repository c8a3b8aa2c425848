"""Device-resident block tables and the step-metadata kernel (csrc/step_meta.hip) against the
host-built metadata of the same cache operations.

Integer work, so the bar is equality.  Two caches see the same operations (alloc, reservation,
decode steps, mixed steps, trims, frees and slot reuse); the host-table cache's metadata is the
reference's arithmetic (kv_cache.py:74-101, pinned on the CPU against oracle.paged.slot_of), the
device-table cache builds its own on the GPU.  Block tables are compared over the entries a row
uses (ceil(kv_len / block_size)); past them the device table holds zeros."""
import math
import random

import pytest
import torch

from conftest import announce
from kv_cache import KVCache
from oracle import paged as opaged

pytestmark = pytest.mark.gpu


def caches(num_blocks=96, max_seqs=12, max_blocks_per_seq=None):
    mk = lambda dt: KVCache(num_blocks, 16, "cuda", torch.bfloat16, 1, 2, 128,  # noqa: E731
                            device_tables=dt, max_seqs=max_seqs,
                            max_blocks_per_seq=max_blocks_per_seq)
    return mk(False), mk(True)


def same_meta(h, d, packed):
    torch.cuda.synchronize()
    assert h.starts == d.starts
    assert torch.equal(h.kv_lens.cpu(), d.kv_lens.cpu())
    assert torch.equal(h.slot_mapping32.cpu(), d.slot_mapping32.cpu())
    kv = h.kv_lens.cpu().tolist()
    hb, db = h.block_table.cpu(), d.block_table.cpu()
    for b, n in enumerate(kv):
        used = math.ceil(n / 16)
        assert torch.equal(hb[b, :used], db[b, :used]), b
        assert not db[b, used:].any()
    if packed:
        for name in ("cu_q", "positions", "last_idx"):
            assert torch.equal(getattr(h, name).cpu(), getattr(d, name).cpu()), name
    else:
        assert torch.equal(h.starts_dev.cpu(), d.starts_dev.cpu())


@pytest.mark.parametrize("cap", [None, 8])
def test_device_metadata_equals_host_metadata_over_a_random_schedule(cap):
    """cap=8: table rows of 8 blocks over a pool of 96, so the device tables' row stride (8) is
    narrower than the pool and the step kernel reads them at that stride."""
    random.seed(0)
    hc, dc = caches(max_blocks_per_seq=cap)
    if cap:
        assert dc.dev_tables.shape[1] == cap < dc.num_blocks
    max_len = (cap or 10**9) * 16
    live = []
    announce(f"[gpu] step metadata: random schedule on host vs device tables, cap {cap}")
    for it in range(60):
        op = random.random()
        if len(live) < 2 or (op < 0.25 and len(live) < 10):
            hs, ds = hc.alloc(), dc.alloc()
            assert hs == ds
            reserve = random.randint(1, min(200, max_len))
            if hc.blocks_needed(hs, reserve) <= hc.free_block_count():
                hc.ensure_capacity(hs, reserve)
                dc.ensure_capacity(ds, reserve)
            live.append(hs)
            continue
        if op < 0.35 and len(live) > 2:
            s = live.pop(random.randrange(len(live)))
            hc.free(s)
            dc.free(s)
            continue
        if op < 0.45:
            s = random.choice(live)
            hc.trim(s)
            dc.trim(s)
            continue
        rows = random.sample(live, random.randint(1, len(live)))
        if op < 0.75:
            T = random.choice([1, 1, 1, 3])
            need = sum(hc.blocks_needed(s, hc.length(s) + T) for s in rows)
            if need > hc.free_block_count() or max(hc.length(s) for s in rows) + T > max_len:
                continue
            h, d = hc.prepare(rows, T), dc.prepare(rows, T)
            same_meta(h, d, packed=False)
            hc.advance(rows, T)
            dc.advance(rows, T)
        else:
            counts = [random.choice([1, 1, 2, 17, 40]) for _ in rows]
            need = sum(hc.blocks_needed(s, hc.length(s) + c) for s, c in zip(rows, counts))
            if need > hc.free_block_count() or any(
                    hc.length(s) + c > max_len for s, c in zip(rows, counts)):
                continue
            h, d = hc.prepare_packed(rows, counts), dc.prepare_packed(rows, counts)
            same_meta(h, d, packed=True)
            hc.advance(rows, counts)
            dc.advance(rows, counts)
        # the device lengths moved with the step, and match the host's
        lens = dc.dev_lens.cpu()
        for s in live:
            assert lens[dc.slot[s]].item() == dc.length(s) == hc.length(s)
    for s in live:
        t = dc._block_tables[s]
        row = dc.dev_tables[dc.slot[s], :len(t)].cpu().tolist()
        assert row == t
        for p in range(dc.length(s)):
            assert opaged.slot_of(t, p, 16) == t[p // 16] * 16 + p % 16


def test_padding_rows_and_rows_past_their_table_are_inert():
    from kernels.meta import step_metadata
    _, dc = caches(num_blocks=8, max_seqs=4)
    a, b = dc.alloc(), dc.alloc()
    dc.ensure_capacity(a, 20)
    dc.ensure_capacity(b, 20)
    # slot b claims 128 held tokens, its whole table row of 8 blocks: one more key would need
    # table entry 8, one past the row (still inside the tables array: the next row's first
    # entry), so the row must be treated as padding
    dc.dev_lens[dc.slot[b]] = 8 * 16
    row_slots = torch.tensor([dc.slot[a], -1, dc.slot[b]], dtype=torch.int32, device="cuda")
    out = torch.full((3 + 3 + 3 * 8 + 3,), 7, dtype=torch.int32, device="cuda")
    announce("[gpu] step metadata: padding and overfull rows")
    step_metadata(dc, row_slots, None, 1, out[:3], out[3:6], out[6:30].view(3, 8), out[30:])
    torch.cuda.synchronize()
    starts, kv, bt, slots = out[:3].tolist(), out[3:6].tolist(), out[6:30].view(3, 8), out[30:].tolist()
    assert kv == [1, 0, 0] and starts[1] == 0
    assert slots[0] == dc._block_tables[a][0] * 16 and slots[1:] == [-1, -1]
    assert not bt[1:].any() and bt[0, 0].item() == dc._block_tables[a][0]
    lens = dc.dev_lens.cpu().tolist()
    assert lens[dc.slot[a]] == 1 and lens[dc.slot[b]] == 8 * 16


def test_graphs_on_device_tables_match_host_tables():
    """The captured decode step over device-resident tables gives the logits of the same step
    captured over host-packed metadata."""
    from graphs import DecodeGraphs
    from model import QwenConfig, Qwen2ForCausalLM
    cfg = QwenConfig(hidden_size=1536, num_layers=2, num_heads=12, num_kv_heads=2, head_dim=128,
                     intermediate_size=1024, vocab_size=512)
    model = Qwen2ForCausalLM(cfg).to("cuda").init_random(std=0.02, seed=0).to(torch.bfloat16).eval()
    outs = []
    g = torch.Generator().manual_seed(8)
    prompts = [torch.randint(0, 512, (1, n), generator=g) for n in (37, 150, 5)]
    toks = torch.randint(0, 512, (3, 3), generator=g)
    for dt in (False, True):
        cache = KVCache(64, 16, "cuda", torch.bfloat16, 2, 2, 128, device_tables=dt)
        announce(f"[gpu] decode graphs, device_tables={dt}")
        graphs = DecodeGraphs(model, cache, buckets=(2, 4))
        seqs = [cache.alloc() for _ in prompts]
        with torch.no_grad():
            for s, p in zip(seqs, prompts):
                model(p.cuda(), cache, [s])
            steps = [graphs.run(seqs, toks[:, t].tolist()).float().clone() for t in range(3)]
        torch.cuda.synchronize()
        outs.append(torch.stack(steps).cpu())
        assert [cache.length(s) for s in seqs] == [40, 153, 8]
    assert torch.equal(outs[0], outs[1])


def _small_model():
    from model import QwenConfig, Qwen2ForCausalLM
    cfg = QwenConfig(hidden_size=1536, num_layers=2, num_heads=12, num_kv_heads=2, head_dim=128,
                     intermediate_size=1024, vocab_size=512)
    return Qwen2ForCausalLM(cfg).to("cuda").init_random(std=0.02, seed=0).to(torch.bfloat16).eval()


def test_graphs_with_tables_narrower_than_the_pool_match_eager_decode():
    """Decode graphs over a cache whose rows hold at most 8 blocks of a 64-block pool: the graphs
    are captured at W = 8 (kv capacity 128 keys, not the pool's 1,024), and their logits equal
    the eager decode's of the same cache state."""
    from graphs import DecodeGraphs
    model = _small_model()
    g = torch.Generator().manual_seed(9)
    prompts = [torch.randint(0, 512, (1, n), generator=g) for n in (37, 100, 5)]
    toks = torch.randint(0, 512, (3, 4), generator=g)
    ec = KVCache(64, 16, "cuda", torch.bfloat16, 2, 2, 128, max_blocks_per_seq=8)
    gc = KVCache(64, 16, "cuda", torch.bfloat16, 2, 2, 128, max_blocks_per_seq=8)
    announce("[gpu] decode graphs over 8-block table rows of a 64-block pool")
    graphs = DecodeGraphs(model, gc, buckets=(2, 4))
    assert graphs.W == 8
    es = [ec.alloc() for _ in prompts]
    gs = [gc.alloc() for _ in prompts]
    with torch.no_grad():
        for p, a, b in zip(prompts, es, gs):
            model(p.cuda(), ec, [a])
            model(p.cuda(), gc, [b])
        for t in range(toks.shape[1]):
            want = model(toks[:, t:t + 1].cuda(), ec, es)[:, -1].float()
            got = graphs.run(gs, toks[:, t].tolist()).float()
            torch.cuda.synchronize()
            assert (got - want).abs().max().item() <= 0.02 * want.abs().max().item(), t
    assert [gc.length(s) for s in gs] == [41, 104, 9]
    assert max(len(gc._block_tables[s]) for s in gs) <= 8


def test_engine_rejects_a_conversation_past_its_table_row_while_blocks_are_free():
    from engine import Engine, run_concurrent_chats
    model = _small_model()
    cache = KVCache(64, 16, "cuda", torch.bfloat16, 2, 2, 128, max_blocks_per_seq=8)
    eng = Engine(model, cache, max_reply_tokens=8, seed=0)
    g = torch.Generator().manual_seed(10)
    # 100 + 8 + 1 tokens fit 8 blocks (128 tokens); 200 + 8 + 1 need 14 blocks of the 8 a row
    # may hold, although 64 blocks are free
    ok, long_ = (torch.randint(0, 512, (n,), generator=g).tolist() for n in (100, 200))
    announce("[gpu] engine: a conversation longer than its table row")
    from engine import Conversation
    c1, c2 = Conversation(), Conversation()
    j1 = eng.submit(c1, ok, 8)
    j2 = eng.submit(c2, long_, 8)
    eng.run_until_idle()
    torch.cuda.synchronize()
    assert j2.rejected and "too long" in j2.rejected and not j2.generated
    assert not j1.rejected and len(j1.generated) == 8
    assert cache.free_block_count() >= 64 - 8

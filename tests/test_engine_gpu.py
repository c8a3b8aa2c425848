"""The Qwen2 model and scheduler on the GPU, attention through libmi_fa2.so's paged kernels,
checked against the same weights run on the CPU in fp32 (the reference model's SDPA fallback)."""
import pytest
import torch

from conftest import announce
from engine import Engine, run_concurrent_chats
from kv_cache import KVCache
from model import QwenConfig, Qwen2ForCausalLM

pytestmark = pytest.mark.gpu

# Qwen2.5's attention shape (12q/2kv, head_dim 128) in a 2-layer model
SMALL = QwenConfig(hidden_size=1536, num_layers=2, num_heads=12, num_kv_heads=2, head_dim=128,
                   intermediate_size=1024, vocab_size=512)


def make(device, dtype, num_blocks=64):
    model = Qwen2ForCausalLM(SMALL).to(device=device, dtype=torch.float32).init_random(std=0.02, seed=0)
    model = model.to(dtype).eval()
    cache = KVCache(num_blocks, 16, device, dtype, SMALL.num_layers, SMALL.num_kv_heads, SMALL.head_dim)
    return model, cache


def test_gpu_paged_model_matches_cpu_fp32():
    g = torch.Generator().manual_seed(1)
    prompts = [torch.randint(0, SMALL.vocab_size, (1, n), generator=g) for n in (37, 150, 5)]
    steps = torch.randint(0, SMALL.vocab_size, (3, 3), generator=g)
    gm, gc = make("cuda", torch.bfloat16)
    cm, cc = make("cpu", torch.float32)
    # identical weights: the CPU model takes the GPU model's bf16 values in fp32
    cm.load_state_dict({k: v.float().cpu() for k, v in gm.state_dict().items()})
    outs = []
    for model, cache, dev in ((gm, gc, "cuda"), (cm, cc, "cpu")):
        seqs = [cache.alloc() for _ in prompts]
        announce(f"[gpu] model prefill+decode on {dev}")
        with torch.no_grad():
            for s, p in zip(seqs, prompts):
                model(p.to(dev), cache, [s])
            for t in range(steps.shape[1]):
                logits = model(steps[:, t:t + 1].to(dev), cache, seqs)
        outs.append(logits.float().cpu())
    torch.cuda.synchronize()
    gpu, cpu = outs
    cos = torch.nn.functional.cosine_similarity(gpu.flatten(), cpu.flatten(), dim=0).item()
    rel = ((gpu - cpu).abs().max() / cpu.abs().max()).item()
    assert cos > 0.999 and rel < 0.05, (cos, rel)


def test_gpu_concurrent_chats_complete():
    model, cache = make("cuda", torch.bfloat16, num_blocks=128)
    eng = Engine(model, cache, max_reply_tokens=8, seed=0)
    g = torch.Generator().manual_seed(2)
    prompts = [torch.randint(0, SMALL.vocab_size, (n,), generator=g).tolist() for n in (40, 7, 300, 96)]
    announce("[gpu] 4 concurrent chats x 8 tokens")
    summary = run_concurrent_chats(eng, prompts, reply_tokens=8)
    assert summary["tokens"] == 32
    assert cache.free_block_count() == 128


def test_captured_decode_graphs_match_eager_decode():
    """Graph replays (padded buckets, static metadata) give the eager decode's logits and cache."""
    from graphs import DecodeGraphs
    g = torch.Generator().manual_seed(3)
    prompts = [torch.randint(0, SMALL.vocab_size, (1, n), generator=g) for n in (37, 150, 5, 64, 20)]
    toks = torch.randint(0, SMALL.vocab_size, (5, 4), generator=g)
    em, ec = make("cuda", torch.bfloat16)
    gm, gc = make("cuda", torch.bfloat16)
    announce("[gpu] decode graphs: capture")
    graphs = DecodeGraphs(gm, gc, buckets=(1, 2, 4, 8))
    es = [ec.alloc() for _ in prompts]
    gs = [gc.alloc() for _ in prompts]
    with torch.no_grad():
        for p, a, b in zip(prompts, es, gs):
            em(p.cuda(), ec, [a])
            gm(p.cuda(), gc, [b])
        # batches of 3, 2 (bucket 2), 5 (bucket 8) and 1 rows
        for t, rows in enumerate(([0, 1, 2], [3, 4], [0, 1, 2, 3, 4], [2])):
            announce(f"[gpu] decode graphs: step {t} rows {rows}")
            want = em(toks[rows, t:t + 1].cuda(), ec, [es[i] for i in rows])[:, -1].float()
            got = graphs.run([gs[i] for i in rows], toks[rows, t].tolist()).float()
            torch.cuda.synchronize()
            scale = want.abs().max().item()
            assert (got - want).abs().max().item() <= 0.02 * scale, t
    assert [ec.length(s) for s in es] == [gc.length(s) for s in gs]
    # the new tokens' K/V went to the same places in both caches (close, not bitwise: the
    # attention outputs of the first layer feed the second layer's projections)
    for i in range(len(prompts)):
        ta, tb = ec._block_tables[es[i]], gc._block_tables[gs[i]]
        n = ec.length(es[i])
        ka = ec.buf[:, :, torch.tensor([ta[p // 16] * 16 + p % 16 for p in range(n)])].float()
        kb = gc.buf[:, :, torch.tensor([tb[p // 16] * 16 + p % 16 for p in range(n)])].float()
        assert (ka - kb).abs().max().item() <= 0.02 * ka.abs().max().item()


def test_engine_with_decode_graphs_completes():
    from graphs import DecodeGraphs
    model, cache = make("cuda", torch.bfloat16, num_blocks=128)
    graphs = DecodeGraphs(model, cache, buckets=(1, 2, 4))
    eng = Engine(model, cache, max_reply_tokens=8, seed=0, decode_graphs=graphs)
    g = torch.Generator().manual_seed(4)
    prompts = [torch.randint(0, SMALL.vocab_size, (n,), generator=g).tolist() for n in (40, 7, 300, 96)]
    announce("[gpu] 4 concurrent chats x 8 tokens, decode graphs")
    summary = run_concurrent_chats(eng, prompts, reply_tokens=8)
    assert summary["tokens"] == 32
    assert cache.free_block_count() == 128


def test_gpu_mixed_step_matches_separate_steps():
    """A packed step (3 decode rows, then prompts of 150, 1 and 40 tokens: the 1-token prompt
    goes through the varlen prefill kernel, not the decode kernel) against the unpacked GPU
    forwards and the CPU fp32 model with the same weights."""
    g = torch.Generator().manual_seed(6)
    hist = [torch.randint(0, SMALL.vocab_size, (n,), generator=g).tolist() for n in (37, 200, 5)]
    nxt = torch.randint(0, SMALL.vocab_size, (3,), generator=g).tolist()
    new = [torch.randint(0, SMALL.vocab_size, (n,), generator=g).tolist() for n in (150, 1, 40)]
    gm, gc = make("cuda", torch.bfloat16)
    cm, cc = make("cpu", torch.float32)
    cm.load_state_dict({k: v.float().cpu() for k, v in gm.state_dict().items()})
    rows = [[t] for t in nxt] + new
    got = {}
    for model, cache, dev in ((gm, gc, "cuda"), (cm, cc, "cpu")):
        seqs = [cache.alloc() for _ in range(6)]
        announce(f"[gpu] mixed step on {dev}: decode rows 3, prompts (150, 1, 40)")
        with torch.no_grad():
            for s, h in zip(seqs, hist):
                model(torch.tensor([h], device=dev), cache, [s])
            got[dev] = model.forward_mixed(rows, cache, seqs).float().cpu()
        assert [cache.length(s) for s in seqs] == [38, 201, 6, 150, 1, 40]
    announce("[gpu] mixed step: unpacked GPU forwards")
    want = []
    with torch.no_grad():
        for r in [h + [t] for h, t in zip(hist, nxt)] + new:
            m2, c2 = gm, KVCache(64, 16, "cuda", torch.bfloat16, SMALL.num_layers,
                                 SMALL.num_kv_heads, SMALL.head_dim)
            want.append(m2(torch.tensor([r], device="cuda"), c2, [c2.alloc()])[:, -1].float().cpu())
    torch.cuda.synchronize()
    want = torch.cat(want)
    gpu, cpu = got["cuda"], got["cpu"]
    scale = cpu.abs().max().item()
    assert (gpu - want).abs().max().item() <= 0.02 * scale
    cos = torch.nn.functional.cosine_similarity(gpu.flatten(), cpu.flatten(), dim=0).item()
    assert cos > 0.999 and (gpu - cpu).abs().max().item() <= 0.05 * scale, cos


def test_engine_mixed_prefill_with_decode_graphs_completes():
    from graphs import DecodeGraphs
    model, cache = make("cuda", torch.bfloat16, num_blocks=128)
    graphs = DecodeGraphs(model, cache, buckets=(1, 2, 4))
    eng = Engine(model, cache, max_reply_tokens=8, seed=0, decode_graphs=graphs, mixed_prefill=True)
    g = torch.Generator().manual_seed(4)
    prompts = [torch.randint(0, SMALL.vocab_size, (n,), generator=g).tolist() for n in (40, 7, 300, 96)]
    announce("[gpu] 4 concurrent chats x 8 tokens, mixed prefill steps + decode graphs")
    summary = run_concurrent_chats(eng, prompts, reply_tokens=8)
    assert summary["tokens"] == 32
    assert cache.free_block_count() == 128


def test_graph_keeps_its_workspace_when_a_later_capture_outgrows_it():
    """Buckets 1 and 8 are captured on one stream: the larger capture needs a larger split-decode
    workspace, and the bucket-1 graph, which holds the first workspace's address, must still
    replay correctly afterwards (an outgrown workspace is kept alive, not freed and reused); and
    no replay may write into memory allocated after the capture (every buffer a graph writes,
    its step-metadata output included, lives as long as the graph)."""
    from graphs import DecodeGraphs
    g = torch.Generator().manual_seed(9)
    prompts = [torch.randint(0, SMALL.vocab_size, (1, n), generator=g) for n in (300, 280, 260, 240,
                                                                                  220, 200, 180, 500)]
    toks = torch.randint(0, SMALL.vocab_size, (8, 3), generator=g)
    em, ec = make("cuda", torch.bfloat16, num_blocks=256)
    gm, gc = make("cuda", torch.bfloat16, num_blocks=256)
    announce("[gpu] decode graphs: buckets 1 and 8 on one capture stream")
    graphs = DecodeGraphs(gm, gc, buckets=(1, 8))
    es = [ec.alloc() for _ in prompts]
    gs = [gc.alloc() for _ in prompts]
    with torch.no_grad():
        for p, a, b in zip(prompts, es, gs):
            em(p.cuda(), ec, [a])
            gm(p.cuda(), gc, [b])
        # churn the allocator so that memory a graph still writes, had it been freed, would be
        # handed to these tensors (small ones share the pool of the graph's metadata buffers)
        junk = [torch.full((1 << 20,), float("nan"), device="cuda") for _ in range(16)]
        junk += [torch.full((2048,), float("nan"), device="cuda") for _ in range(512)]
        for t, rows in enumerate(([7], list(range(8)), [7])):
            want = em(toks[rows, t:t + 1].cuda(), ec, [es[i] for i in rows])[:, -1].float()
            got = graphs.run([gs[i] for i in rows], toks[rows, t].tolist()).float()
            torch.cuda.synchronize()
            assert torch.isfinite(got).all() and torch.isfinite(want).all(), t
            assert (got - want).abs().max().item() <= 0.02 * want.abs().max().item(), t
        # no replay wrote into memory the graphs do not own
        assert all(torch.isnan(j).all().item() for j in junk)
        del junk

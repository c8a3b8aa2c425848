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

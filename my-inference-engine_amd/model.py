"""Qwen2-architecture causal LM whose attention runs on the MI355X paged kernels.

Mirrors the reference's model.py (Qwen2ForCausalLM, model.py:141-207) layer for layer -- fp32
RMSNorm (model.py:43-55), rotate-half RoPE with theta 1e6 (model.py:58-65,148-155), biased q/k/v
projections (model.py:81-84), SwiGLU MLP (model.py:112-120), tied embeddings and last-position
logits (model.py:204-207) -- with two deliberate differences on the GPU path:

  * Attention reads K/V straight from the paged cache inside the kernel (kernels.fa2.fa2_paged)
    instead of gathering a dense copy every layer of every step (KVCache.read, kv_cache.py:117-121,
    called at model.py:97) and then calling the padded kernel (model.py:103).
  * The q/k/v and gate/up projections are single fused GEMMs (one launch instead of three/two).
  * RoPE and the cache write are one HIP launch (kernels.rope.rope_kv_write) instead of the
    elementwise RoPE ops and two index_copy_ (model.py:92,96), with bitwise the same results.

On CPU tensors the model takes the reference's own fallback (dense read + fp32 SDPA with the
bottom-right mask, model.py:104-107,181-195), which only the CPU tests of the scheduler use; the
attention kernels themselves have no CPU path.
"""
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from kernels.fa2 import fa2_paged
from kernels.rope import rope_kv_write


@dataclass(frozen=True)
class QwenConfig:
    hidden_size: int = 1536
    num_layers: int = 28
    num_heads: int = 12
    num_kv_heads: int = 2
    head_dim: int = 128
    intermediate_size: int = 8960
    vocab_size: int = 151936
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0


QWEN25_1P5B = QwenConfig()  # model.py:18-27


class RMSNorm(nn.Module):
    """Normalise in fp32, scale in the input dtype (model.py:49-55)."""

    def __init__(self, dim, eps):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x):
        dtype = x.dtype
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return self.weight * xf.to(dtype)


def rotate_half(x):
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


def apply_rope(q, k, cos, sin):
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


def repeat_kv(x, n_rep):
    if n_rep == 1:
        return x
    b, h, s, d = x.shape
    return x[:, :, None].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)


class Attention(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.cfg = cfg
        self.q_size = cfg.num_heads * cfg.head_dim
        self.kv_size = cfg.num_kv_heads * cfg.head_dim
        self.qkv_proj = nn.Linear(cfg.hidden_size, self.q_size + 2 * self.kv_size, bias=True)
        self.o_proj = nn.Linear(self.q_size, cfg.hidden_size, bias=False)

    def forward(self, x, cos, sin, cache, layer, meta):
        cfg = self.cfg
        B, T, _ = x.shape
        qkv = self.qkv_proj(x)
        if x.is_cuda:
            # rotated q out, rotated k and v into their cache slots, in one launch
            q = rope_kv_write(qkv.view(B * T, -1), cos[:, 0].reshape(B * T, cfg.head_dim),
                              sin[:, 0].reshape(B * T, cfg.head_dim), meta.slot_mapping32,
                              cache.k_pool(layer), cache.v_pool(layer), cfg.num_heads,
                              cfg.num_kv_heads)
            q = q.view(B, T, cfg.num_heads, cfg.head_dim).transpose(1, 2)
            out = fa2_paged(q, cache.k_pool(layer), cache.v_pool(layer), meta.block_table,
                            meta.kv_lens, block_size=cache.block_size, max_kv_len=meta.max_kv,
                            is_causal=T > 1)
        else:
            q, k, v = qkv.split([self.q_size, self.kv_size, self.kv_size], dim=-1)
            q = q.view(B, T, cfg.num_heads, cfg.head_dim).transpose(1, 2)
            k = k.view(B, T, cfg.num_kv_heads, cfg.head_dim).transpose(1, 2)
            v = v.view(B, T, cfg.num_kv_heads, cfg.head_dim).transpose(1, 2)
            q, k = apply_rope(q, k, cos, sin)
            cache.write(layer, meta, k, v)
            k_all, v_all = cache.read(layer, meta)
            n_rep = cfg.num_heads // cfg.num_kv_heads
            out = F.scaled_dot_product_attention(q, repeat_kv(k_all, n_rep), repeat_kv(v_all, n_rep),
                                                 attn_mask=meta.dense_mask(x.device))
        return self.o_proj(out.transpose(1, 2).reshape(B, T, self.q_size))


class MLP(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.inter = cfg.intermediate_size
        self.gate_up_proj = nn.Linear(cfg.hidden_size, 2 * cfg.intermediate_size, bias=False)
        self.down_proj = nn.Linear(cfg.intermediate_size, cfg.hidden_size, bias=False)

    def forward(self, x):
        gate, up = self.gate_up_proj(x).split(self.inter, dim=-1)
        return self.down_proj(F.silu(gate) * up)


class Block(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.self_attn = Attention(cfg)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.mlp = MLP(cfg)

    def forward(self, x, cos, sin, cache, layer, meta):
        x = x + self.self_attn(self.input_layernorm(x), cos, sin, cache, layer, meta)
        return x + self.mlp(self.post_attention_layernorm(x))


class Qwen2ForCausalLM(nn.Module):
    def __init__(self, cfg=QWEN25_1P5B):
        super().__init__()
        self.cfg = cfg
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList(Block(cfg) for _ in range(cfg.num_layers))
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        inv_freq = 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.head_dim, 2).float() / cfg.head_dim))
        self.register_buffer("inv_freq", inv_freq, persistent=False)

    @torch.no_grad()
    def init_random(self, std=0.02, seed=0):
        """Random weights: N(0, std) for every matrix and bias, ones for the norms."""
        g = torch.Generator(device=self.embed_tokens.weight.device).manual_seed(seed)
        for name, prm in self.named_parameters():
            if name.endswith("layernorm.weight") or name == "norm.weight":
                prm.fill_(1.0)
            else:
                prm.copy_(torch.randn(prm.shape, generator=g, device=prm.device,
                                      dtype=torch.float32).mul_(std).to(prm.dtype))
        return self

    def rope_cos_sin(self, position_ids, dtype):
        # position_ids [B, T] -> cos/sin [B, 1, T, head_dim] (model.py:151-155)
        freqs = position_ids.float()[..., None] * self.inv_freq[None, None, :]
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos()[:, None].to(dtype), emb.sin()[:, None].to(dtype)

    def forward(self, input_ids, cache, seqs):
        """input_ids [B, T] appended to cache sequences `seqs`; returns last-position logits
        [B, 1, vocab] (model.py:157-207)."""
        _, T = input_ids.shape
        meta = cache.prepare(seqs, T)
        logits = self.forward_meta(input_ids, cache, meta)
        cache.advance(seqs, T)
        return logits

    def forward_meta(self, input_ids, cache, meta):
        """The layers over an already prepared step: what a captured decode graph replays, its
        metadata living in static device buffers."""
        _, T = input_ids.shape
        x = self.embed_tokens(input_ids)
        position_ids = meta.starts_dev[:, None] + torch.arange(T, device=x.device)[None, :]
        cos, sin = self.rope_cos_sin(position_ids, x.dtype)
        for layer_idx, layer in enumerate(self.layers):
            x = layer(x, cos, sin, cache, layer_idx, meta)
        x = self.norm(x[:, -1:])
        return x @ self.embed_tokens.weight.T

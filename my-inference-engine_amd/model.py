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
  * Each residual add and the RMSNorm after it are one HIP launch (kernels.model_ops.add_rmsnorm)
    and SiLU x up is one more (kernels.model_ops.silu_mul), instead of about twenty small torch
    launches per layer, with the same rounding points.
  * The gate/up GEMM and the tied lm_head multiply by a cached transposed copy of their weight
    ([in, out] row-major): at decode sizes hipBLASLt picks much faster kernels for that layout of
    these two shapes (the other projections are faster as they are).  The parameters keep the
    reference's layout; the copy is rebuilt if a weight changes.

forward_mixed() runs one step over rows that append different numbers of tokens -- decoding chats
(one token each) and newly admitted prompts -- packed back to back: every projection, norm and MLP
runs once over all packed tokens, attention goes to the paged decode kernel for the leading
one-token rows and to the paged varlen prefill kernel for the prompt rows, and only each row's last
token reaches the logits.  The reference runs each admitted prompt as a forward of its own
(chat.py:157-185, one per tick, chat.py:247-253) beside the batched decode step.

On CPU tensors the model takes the reference's own fallback (dense read + fp32 SDPA with the
bottom-right mask, model.py:104-107,181-195), which only the CPU tests of the scheduler use; the
attention kernels themselves have no CPU path.
"""
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from kernels.fa2 import fa2_paged, fa2_paged_varlen
from kernels.model_ops import add_rmsnorm, silu_mul
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
        if x.is_cuda:
            shape = x.shape
            return add_rmsnorm(x.reshape(-1, shape[-1]), self.weight, self.eps)[1].view(shape)
        dtype = x.dtype
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return self.weight * xf.to(dtype)


def rotate_half(x):
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


def apply_rope(q, k, cos, sin):
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


def transposed(weight):
    """weight.t().contiguous(), cached on the parameter and rebuilt when it is modified."""
    cached = getattr(weight, "_mi_transposed", None)
    if cached is None or cached[0] != weight._version:
        cached = (weight._version, weight.detach().t().contiguous())
        weight._mi_transposed = cached
    return cached[1]


def repeat_kv(x, n_rep):
    if n_rep == 1:
        return x
    b, h, s, d = x.shape
    return x[:, :, None].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)


def sdpa_fallback(q, k, v, starts, n_rep):
    """The reference's CPU attention: fp32 SDPA over repeat_kv-expanded K/V (model.py:104-107)
    with its mask choice (model.py:181-195).  q [B, Hq, T, d], k/v [B, Hkv, S, d] dense (every row
    padded to S keys); starts[b]: tokens row b held before this step.  When every row starts at
    the same place no mask is built: a fresh prefill (start 0) is SDPA's is_causal, whose top-left
    alignment equals the bottom-right one when T == S, and a one-token step sees every key.
    Otherwise the explicit [B, 1, T, S] bottom-right mask: query i of row b sees key j iff
    j <= starts[b] + i."""
    T, S = q.shape[2], k.shape[2]
    k, v = repeat_kv(k, n_rep), repeat_kv(v, n_rep)
    c0 = starts[0]
    if all(st == c0 for st in starts) and (T == 1 or c0 == 0):
        return F.scaled_dot_product_attention(q, k, v, is_causal=c0 == 0)
    key_pos = torch.arange(S, device=q.device)
    q_pos = (torch.tensor(starts, device=q.device)[:, None]
             + torch.arange(T, device=q.device)[None, :])
    mask = (key_pos[None, None, :] <= q_pos[:, :, None]).unsqueeze(1)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask)


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
            if meta.packed:
                out = self._attend_packed(q.view(B * T, cfg.num_heads, cfg.head_dim), cache,
                                          layer, meta)
                return self.o_proj(out.view(B, T, self.q_size))
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
            if meta.packed:
                out = self._attend_packed_cpu(q, cache, layer, meta)
                return self.o_proj(out.transpose(1, 2).reshape(B, T, self.q_size))
            k_all, v_all = cache.read(layer, meta)
            out = sdpa_fallback(q, k_all, v_all, meta.starts, cfg.num_heads // cfg.num_kv_heads)
        return self.o_proj(out.transpose(1, 2).reshape(B, T, self.q_size))

    def _attend_packed(self, q, cache, layer, meta):
        """q [N, Hq, d] packed queries of a mixed step -> [N, Hq, d]: the leading one-token rows
        through the paged decode kernel, the rest through the paged varlen prefill kernel, both
        writing into one packed output."""
        out = torch.empty_like(q)
        D, B, bs = meta.n_single, len(meta.counts), cache.block_size
        kv_single, kv_multi, q_multi = meta.split()
        kp, vp = cache.k_pool(layer), cache.v_pool(layer)
        if D:
            fa2_paged(q[:D].unsqueeze(2), kp, vp, meta.block_table[:D], meta.kv_lens[:D],
                      block_size=bs, max_kv_len=kv_single, is_causal=False,
                      out=out[:D].unsqueeze(2))
        if D < B:
            fa2_paged_varlen(q, kp, vp, meta.cu_q[D:], meta.block_table[D:], meta.kv_lens[D:],
                             q_multi, block_size=bs, max_kv_len=kv_multi, is_causal=True, out=out)
        return out

    def _attend_packed_cpu(self, q, cache, layer, meta):
        """The dense fallback row by row: q [1, Hq, N, d] -> [1, Hq, N, d] (model.py:181-195)."""
        n_rep = self.cfg.num_heads // self.cfg.num_kv_heads
        outs, c0 = [], 0
        for start, count, table in zip(meta.starts, meta.counts, meta.tables):
            k_all, v_all = cache.read_row(layer, table, start + count)
            mask = (torch.arange(start + count, device=q.device)[None, :]
                    <= start + torch.arange(count, device=q.device)[:, None])
            outs.append(F.scaled_dot_product_attention(
                q[:, :, c0:c0 + count], repeat_kv(k_all[None], n_rep), repeat_kv(v_all[None], n_rep),
                attn_mask=mask))
            c0 += count
        return torch.cat(outs, dim=2)


class MLP(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.inter = cfg.intermediate_size
        self.gate_up_proj = nn.Linear(cfg.hidden_size, 2 * cfg.intermediate_size, bias=False)
        self.down_proj = nn.Linear(cfg.intermediate_size, cfg.hidden_size, bias=False)

    def forward(self, x):
        if x.is_cuda:
            gu = x.reshape(-1, x.shape[-1]) @ transposed(self.gate_up_proj.weight)
            act = silu_mul(gu).view(*x.shape[:-1], self.inter)
            return self.down_proj(act)
        gu = self.gate_up_proj(x)
        gate, up = gu.split(self.inter, dim=-1)
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
        x = self.run_layers(x, cos, sin, cache, meta)
        x = self.norm(x[:, -1:])
        return self.lm_head(x)

    def lm_head(self, x):
        """Tied-embedding logits (model.py:204-207)."""
        if x.is_cuda:
            return x @ transposed(self.embed_tokens.weight)
        return x @ self.embed_tokens.weight.T

    def run_layers(self, x, cos, sin, cache, meta):
        """The decoder layers over x [B, T, hidden].  On the GPU each residual add is fused with the
        RMSNorm that follows it (the first layer's input norm has no add; the last layer's MLP
        output is added alone), which is the same arithmetic as Block.forward layer by layer."""
        if not x.is_cuda:
            for layer_idx, layer in enumerate(self.layers):
                x = layer(x, cos, sin, cache, layer_idx, meta)
            return x
        shape, H, eps = x.shape, x.shape[-1], self.cfg.rms_norm_eps
        res = x.reshape(-1, H)
        _, h = add_rmsnorm(res, self.layers[0].input_layernorm.weight, eps)
        for i, layer in enumerate(self.layers):
            a = layer.self_attn(h.view(shape), cos, sin, cache, i, meta).reshape(-1, H)
            res, h = add_rmsnorm(res, layer.post_attention_layernorm.weight, eps, y=a,
                                 residual_out=res)
            m = layer.mlp(h.view(shape)).reshape(-1, H)
            if i + 1 < len(self.layers):
                res, h = add_rmsnorm(res, self.layers[i + 1].input_layernorm.weight, eps, y=m,
                                     residual_out=res)
            else:
                res = res + m
        return res.view(shape)

    def forward_mixed(self, rows, cache, seqs):
        """One packed step: rows[b] (a list of token ids, at least one) is appended to cache
        sequence seqs[b].  Returns each row's last-token logits [B, vocab]."""
        counts = [len(r) for r in rows]
        meta = cache.prepare_packed(seqs, counts)
        ids = torch.tensor([t for r in rows for t in r], dtype=torch.long)
        if cache.device.type == "cuda":
            ids = ids.pin_memory().to(cache.device, non_blocking=True)
        logits = self.forward_packed(ids, cache, meta)
        cache.advance(seqs, counts)
        return logits

    def forward_packed(self, token_ids, cache, meta):
        """The layers over a prepared mixed step (KVCache.prepare_packed): token_ids [N] are the
        rows' new tokens back to back; returns the rows' last-token logits [B, vocab]."""
        x = self.embed_tokens(token_ids)[None]                      # [1, N, hidden]
        cos, sin = self.rope_cos_sin(meta.positions[None], x.dtype)
        x = self.run_layers(x, cos, sin, cache, meta)
        x = self.norm(x[0, meta.last_idx.long()])
        return self.lm_head(x)

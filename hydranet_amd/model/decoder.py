"""Mixtral-shaped decoder around the gfx950 MoE layer: the whole-model decode
harness.

Attention, RoPE, RMSNorm, embeddings and the LM head are stock PyTorch fp16
(they are not the INT4 expert path); every MoE block is MixtralMoELayer on the
gfx950 kernels with its experts resident in HBM.  Structure and arithmetic
follow the reference:

* RMSNorm in fp32, scaled by the weight, cast back (model/mixtral.py:23-37);
* RoPE with a cos/sin cache, rotate_half (model/mixtral.py:40-101);
* grouped-query attention, softmax in fp32 (model/mixtral.py:104-229);
* block = x + attn(norm(x)), then + moe(norm(.)) (model/mixtral.py:373-427);
* a preallocated per-layer KV cache [B, kv_heads, max_len, head_dim] with one
  length for the whole batch (cache/kv_cache.py:26-284, SimpleKVCache);
* top-2 routing at prefill, top-1 or top-2 at decode (TopKMode,
  model/mixtral.py:493-531; the reference's default is top-1 at decode).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .moe import MixtralMoELayer


@dataclass
class MixtralDecoderConfig:
    """Mixtral-8x7B shapes (config.py MixtralConfig of the reference)."""
    num_layers: int = 32
    hidden_dim: int = 4096
    intermediate_dim: int = 14336
    num_attention_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128
    vocab_size: int = 32000
    num_experts: int = 8
    experts_per_token: int = 2
    rms_norm_eps: float = 1e-5
    rope_theta: float = 1e6
    max_position_embeddings: int = 32768
    group_size: int = 128


class RMSNorm(nn.Module):
    def __init__(self, hidden_dim: int, eps: float = 1e-5):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        dt = x.dtype
        x = x.to(torch.float32)
        x = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps)
        return (self.weight * x).to(dt)


class RotaryEmbedding(nn.Module):
    def __init__(self, dim: int, max_positions: int, base: float, device=None):
        super().__init__()
        inv = 1.0 / (base ** (torch.arange(0, dim, 2, device=device).float() / dim))
        t = torch.arange(max_positions, device=device, dtype=torch.float32)
        emb = torch.cat([torch.outer(t, inv)] * 2, dim=-1)
        self.register_buffer("cos_cached", emb.cos(), persistent=False)
        self.register_buffer("sin_cached", emb.sin(), persistent=False)

    def forward(self, position_ids: torch.Tensor):
        # [B, S] -> [B, 1, S, head_dim], broadcast over heads
        return (self.cos_cached[position_ids].unsqueeze(1),
                self.sin_cached[position_ids].unsqueeze(1))


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rotary(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


class KVCache:
    """Preallocated K/V per layer, [B, kv_heads, max_len, head_dim], one
    current length for the whole batch (SimpleKVCache's fp16 mode)."""

    def __init__(self, num_layers: int, batch: int, num_kv_heads: int, head_dim: int,
                 max_len: int, device, dtype=torch.float16):
        shape = (batch, num_kv_heads, max_len, head_dim)
        self.k = [torch.zeros(shape, device=device, dtype=dtype) for _ in range(num_layers)]
        self.v = [torch.zeros(shape, device=device, dtype=dtype) for _ in range(num_layers)]
        self.max_len = max_len
        self.cur_len = 0

    def update(self, layer: int, k: torch.Tensor, v: torch.Tensor, start: int) -> None:
        end = start + k.shape[2]
        assert end <= self.max_len, f"KV cache full ({end} > {self.max_len})"
        self.k[layer][:, :, start:end] = k
        self.v[layer][:, :, start:end] = v

    def get(self, layer: int, total: int):
        return self.k[layer][:, :, :total], self.v[layer][:, :, :total]

    def advance(self, n: int) -> None:
        self.cur_len += n

    def reset(self) -> None:
        self.cur_len = 0


class Attention(nn.Module):
    """Grouped-query attention with RoPE and the KV cache; scores and softmax
    as the reference computes them (fp16 products, fp32 softmax)."""

    def __init__(self, cfg: MixtralDecoderConfig, device=None):
        super().__init__()
        self.nh, self.nkv, self.hd = cfg.num_attention_heads, cfg.num_kv_heads, cfg.head_dim
        H = cfg.hidden_dim
        self.q_proj = nn.Linear(H, self.nh * self.hd, bias=False)
        self.k_proj = nn.Linear(H, self.nkv * self.hd, bias=False)
        self.v_proj = nn.Linear(H, self.nkv * self.hd, bias=False)
        self.o_proj = nn.Linear(self.nh * self.hd, H, bias=False)
        self.rope = RotaryEmbedding(self.hd, cfg.max_position_embeddings, cfg.rope_theta, device)

    def forward(self, x: torch.Tensor, position_ids: torch.Tensor, cache: KVCache,
                layer: int) -> torch.Tensor:
        B, S, _ = x.shape
        q = self.q_proj(x).view(B, S, self.nh, self.hd).transpose(1, 2)
        k = self.k_proj(x).view(B, S, self.nkv, self.hd).transpose(1, 2)
        v = self.v_proj(x).view(B, S, self.nkv, self.hd).transpose(1, 2)
        cos, sin = self.rope(position_ids)
        q, k = apply_rotary(q, k, cos.to(q.dtype), sin.to(q.dtype))
        start = cache.cur_len
        cache.update(layer, k, v, start)
        kf, vf = cache.get(layer, start + S)
        rep = self.nh // self.nkv
        kf = kf.repeat_interleave(rep, dim=1)  # contiguous [B, nh, L, hd]
        vf = vf.repeat_interleave(rep, dim=1)
        scores = torch.matmul(q.contiguous(), kf.transpose(2, 3).contiguous()) / math.sqrt(self.hd)
        if S > 1:  # causal over the new tokens (positions start .. start + S - 1)
            L = start + S
            mask = torch.full((S, L), float("-inf"), device=x.device, dtype=scores.dtype)
            mask = torch.triu(mask, diagonal=start + 1)
            scores = scores + mask
        p = F.softmax(scores, dim=-1, dtype=torch.float32).to(q.dtype)
        o = torch.matmul(p, vf)
        return self.o_proj(o.transpose(1, 2).reshape(B, S, self.nh * self.hd))


class DecoderBlock(nn.Module):
    def __init__(self, cfg: MixtralDecoderConfig, layer_idx: int, slots, device=None):
        super().__init__()
        self.layer_idx = layer_idx
        self.input_layernorm = RMSNorm(cfg.hidden_dim, cfg.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_dim, cfg.rms_norm_eps)
        self.self_attn = Attention(cfg, device)
        self.moe = MixtralMoELayer(cfg.hidden_dim, cfg.num_experts, cfg.experts_per_token,
                                   layer_idx=layer_idx, slots=slots)

    def forward(self, x, position_ids, cache: KVCache, top_k: int):
        x = x + self.self_attn(self.input_layernorm(x), position_ids, cache, self.layer_idx)
        return x + self.moe(self.post_attention_layernorm(x), top_k=top_k)


class MixtralDecoder(nn.Module):
    """Embeddings -> blocks -> norm -> LM head (model/mixtral.py:430-599), with
    every expert resident (one GpuExpertSlot per expert, `slots[layer][e]`)."""

    def __init__(self, cfg: MixtralDecoderConfig, slots: List[list], device=None,
                 decode_top_k: int = 1):
        super().__init__()
        self.cfg = cfg
        self.decode_top_k = decode_top_k
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_dim)
        self.layers = nn.ModuleList([DecoderBlock(cfg, i, slots[i], device)
                                     for i in range(cfg.num_layers)])
        self.norm = RMSNorm(cfg.hidden_dim, cfg.rms_norm_eps)
        self.lm_head = nn.Linear(cfg.hidden_dim, cfg.vocab_size, bias=False)

    def new_cache(self, batch: int, max_len: int) -> KVCache:
        dev = self.embed_tokens.weight.device
        return KVCache(self.cfg.num_layers, batch, self.cfg.num_kv_heads, self.cfg.head_dim,
                       max_len, dev, self.embed_tokens.weight.dtype)

    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor, cache: KVCache,
                top_k: Optional[int] = None) -> torch.Tensor:
        """input_ids [B, S] -> logits [B, S, vocab]; appends S positions to the
        cache (prefill when it is empty: top-2; decode: decode_top_k)."""
        B, S = input_ids.shape
        if top_k is None:
            top_k = 2 if cache.cur_len == 0 else self.decode_top_k
        pos = torch.arange(cache.cur_len, cache.cur_len + S, device=input_ids.device)
        pos = pos.unsqueeze(0).expand(B, S)
        x = self.embed_tokens(input_ids)
        for blk in self.layers:
            x = blk(x, pos, cache, top_k)
        cache.advance(S)
        return self.lm_head(self.norm(x))

    @torch.no_grad()
    def generate_greedy(self, input_ids: torch.Tensor, max_new_tokens: int,
                        cache: Optional[KVCache] = None) -> torch.Tensor:
        """Greedy (top-1 token) decode of max_new_tokens after the prompt; the
        batch shares one length (uniform prompts, no early stop)."""
        B, S = input_ids.shape
        if cache is None:
            cache = self.new_cache(B, S + max_new_tokens)
        logits = self.forward(input_ids, cache)
        tok = logits[:, -1].argmax(-1, keepdim=True)
        out = [tok]
        for _ in range(max_new_tokens - 1):
            logits = self.forward(tok, cache)
            tok = logits[:, -1].argmax(-1, keepdim=True)
            out.append(tok)
        return torch.cat(out, dim=1)


def build_synthetic_decoder(cfg: MixtralDecoderConfig, device="cuda", decode_top_k: int = 1,
                            seed: int = 0) -> MixtralDecoder:
    """Random-init decoder of cfg's shape: dense weights N(0, 0.02) fp16 (the
    reference tests' recipe), norms 1, every expert N(0, 0.02) quantised to
    INT4 by the GPU packer (per-expert seed 42 + layer * 100 + expert) and
    resident in HBM."""
    from ..preprocess.synthetic import expert_seed, make_expert_slot
    dev = torch.device(device)
    slots = [[make_expert_slot(expert_seed(l, e), cfg.hidden_dim, cfg.intermediate_dim,
                               cfg.group_size, device=dev, slot_idx=e)
              for e in range(cfg.num_experts)] for l in range(cfg.num_layers)]
    with torch.device(dev):  # dense modules allocated on the GPU, not initialised on the host
        m = MixtralDecoder(cfg, slots, device=dev, decode_top_k=decode_top_k)
    m = m.to(device=dev, dtype=torch.float16)
    g = torch.Generator(device=dev).manual_seed(seed)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if name.endswith("norm.weight") or "layernorm" in name:
                p.fill_(1.0)
            else:
                p.copy_((torch.randn(p.shape, generator=g, device=dev) * 0.02).to(p.dtype))
    m.eval()
    return m

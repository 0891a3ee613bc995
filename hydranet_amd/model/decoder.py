"""Mixtral-shaped decoder around the gfx950 MoE layer: the whole-model decode
harness (64 sequences of the Mixtral-8x7B shape, decode tokens/s).

Every MoE block is MixtralMoELayer on the gfx950 kernels with its experts
resident in HBM.  Around it, on the GPU: RMSNorm (with the router logits of
its rows, and with the MoE block's unpermute folded in) and, for one-token
decode steps, RoPE + cache append + attention in one launch are library
kernels; the q/k/v, o and LM-head products, embeddings and prefill
attention are PyTorch fp16 (hipBLASLt).  Structure and arithmetic follow the
reference:

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

import numpy as np
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

    def forward(self, pos: torch.Tensor):
        """pos [S] -> cos, sin [S, head_dim] (broadcast over batch and heads)."""
        return self.cos_cached[pos], self.sin_cached[pos]


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rotary(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


class KVCache:
    """Preallocated K/V per layer with one current length for the whole batch
    (SimpleKVCache's fp16 mode).  Keys are stored transposed,
    kt[layer] = [B, kv_heads, head_dim, max_len], so the score product reads
    them as a row-major right operand; values as v[layer] = [B, kv_heads,
    max_len, head_dim].  Writes go to positions given as a device tensor, which
    lets a captured decode step write where its position counter points."""

    def __init__(self, num_layers: int, batch: int, num_kv_heads: int, head_dim: int,
                 max_len: int, device, dtype=torch.float16):
        self.kt = [torch.zeros((batch, num_kv_heads, head_dim, max_len), device=device,
                               dtype=dtype) for _ in range(num_layers)]
        self.v = [torch.zeros((batch, num_kv_heads, max_len, head_dim), device=device,
                              dtype=dtype) for _ in range(num_layers)]
        self.max_len = max_len
        self.cur_len = 0

    def update(self, layer: int, k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor) -> None:
        """k, v [B, kv_heads, S, head_dim] at positions pos [S] (int64, on the device)."""
        self.kt[layer].index_copy_(3, pos, k.transpose(2, 3))
        self.v[layer].index_copy_(2, pos, v)

    def get(self, layer: int, total: int):
        """(K^T [B, kvh, hd, total], V [B, kvh, total, hd]) views of the first positions."""
        return self.kt[layer][..., :total], self.v[layer][:, :, :total]

    def advance(self, n: int) -> None:
        self.cur_len += n
        assert self.cur_len <= self.max_len, f"KV cache full ({self.cur_len} > {self.max_len})"

    def reset(self) -> None:
        self.cur_len = 0


class Attention(nn.Module):
    """Grouped-query attention over the KV cache; scores and softmax as the
    reference computes them (fp16 products scaled by 1/sqrt(head_dim), fp32
    softmax).  The query heads that share a KV head are stacked as the rows of
    one product with that head's keys (head h uses KV head h // (heads /
    kv_heads), as repeat_interleave gives), so the cache is never expanded."""

    def __init__(self, cfg: MixtralDecoderConfig):
        super().__init__()
        self.nh, self.nkv, self.hd = cfg.num_attention_heads, cfg.num_kv_heads, cfg.head_dim
        H = cfg.hidden_dim
        self.q_proj = nn.Linear(H, self.nh * self.hd, bias=False)
        self.k_proj = nn.Linear(H, self.nkv * self.hd, bias=False)
        self.v_proj = nn.Linear(H, self.nkv * self.hd, bias=False)
        self.o_proj = nn.Linear(self.nh * self.hd, H, bias=False)
        # one-token steps on the GPU: attention in one launch (hn_attn_decode)
        # where its shape limits allow; False keeps the two products
        self.decode_kernel = True

    def _decode_fits(self, x: torch.Tensor, S: int, cache: "KVCache", kv_len: int,
                     mask: Optional[torch.Tensor]) -> bool:
        return (self.decode_kernel and x.is_cuda and S == 1 and self.hd == 128
                and self.nh // self.nkv in (1, 2, 4) and 1 <= kv_len <= 1024
                and cache.max_len % 8 == 0 and cache.max_len >= -(-kv_len // 8) * 8
                and (mask is None or (mask.dtype == torch.float16 and mask.numel() == kv_len
                                      and mask.is_contiguous())))

    def _qkv(self, x2: torch.Tensor) -> torch.Tensor:
        """q, k and v projections of x2 [rows, H] as one product: the fp16
        weights stacked into one matrix (one GEMM), or, for Int4Linear
        projections (convert_dense_to_int4), their packed weights and scales
        stacked into one hn_int4_linear launch.  The stack is rebuilt when a
        weight is replaced or modified."""
        from ..kernels.int4_linear import Int4Linear, stacked_int4
        projs = (self.q_proj, self.k_proj, self.v_proj)
        int4 = all(isinstance(m, Int4Linear) for m in projs)
        ts = [t for m in projs for t in ((m.weight_packed, m.weight_scale) if int4 else
                                         (m.weight,))]
        key = (int4,) + tuple((t.data_ptr(), t._version) for t in ts)
        if getattr(self, "_qkv_key", None) != key:
            if int4:
                assert all(m.bias is None for m in projs), "q/k/v projections carry no bias"
                self._qkv_w = stacked_int4(projs)
            else:
                self._qkv_w = torch.cat([m.weight.detach() for m in projs], 0)
            self._qkv_key = key
        if int4:
            from ..kernels.int4_gemm import int4_linear
            packed, scale, g = self._qkv_w
            return int4_linear(x2, packed, scale, g)
        return F.linear(x2, self._qkv_w)

    def forward(self, x: torch.Tensor, rope: "RotaryEmbedding", pos: torch.Tensor,
                cache: KVCache, layer: int, kv_len: int,
                mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x [B, S, H]; tokens at positions pos [S] (int64, x's device);
        attends over the cache's first kv_len positions, adding mask
        [S, kv_len] (0 / -inf) when given.  On the GPU the projections run
        as one GEMM and RoPE + the cache append as one kernel
        (hn_rope_append); on the CPU, the same steps in torch."""
        B, S, _ = x.shape
        nh, nkv, hd = self.nh, self.nkv, self.hd
        rep = nh // nkv
        if x.is_cuda:
            from .. import _lib
            # positions are < cache.max_len (checked by the callers), so the
            # RoPE table rows read are in range
            assert cache.max_len <= rope.cos_cached.shape[0], "RoPE table shorter than the cache"
            assert x.dtype == torch.float16 and pos.dtype == torch.int64
            # the kernel reads fp32 tables (a module-wide .half() would have cast them)
            cos_t = rope.cos_cached.float().contiguous()
            sin_t = rope.sin_cached.float().contiguous()
            qkv = self._qkv(x.reshape(B * S, -1))
            if self._decode_fits(x, S, cache, kv_len, mask) and qkv.stride(-1) == 1 \
                    and qkv.stride(0) % 2 == 0 and qkv.data_ptr() % 4 == 0:
                # one-token step: RoPE, the cache append and attention in one
                # launch (hn_attn_decode_rope)
                o = torch.empty((B, nh * hd), dtype=x.dtype, device=x.device)
                inv = float(np.float32(1.0) / np.float32(math.sqrt(hd)))
                _lib.call("hn_attn_decode_rope", _lib.ptr(qkv), qkv.stride(0), _lib.ptr(cos_t),
                          _lib.ptr(sin_t), _lib.ptr(pos), _lib.ptr(cache.kt[layer]),
                          _lib.ptr(cache.v[layer]), cache.max_len, B, nkv, rep, hd, kv_len,
                          _lib.ptr(mask), inv, _lib.ptr(o), o.stride(0), _lib.stream(x.device))
                return self.o_proj(o.view(B, S, nh * hd))
            wq, wk = nh * hd, nkv * hd
            qg = torch.empty((B, nkv, rep * S, hd), dtype=x.dtype, device=x.device)
            ld = qkv.stride(0)
            base = qkv.data_ptr()
            _lib.call("hn_rope_append", base, ld, base + 2 * wq, ld, base + 2 * (wq + wk), ld,
                      _lib.ptr(cos_t), _lib.ptr(sin_t), _lib.ptr(pos), B, S,
                      nh, nkv, hd, _lib.ptr(qg), _lib.ptr(cache.kt[layer]),
                      _lib.ptr(cache.v[layer]), cache.max_len, _lib.stream(x.device))
        else:
            q = self.q_proj(x).view(B, S, nh, hd).transpose(1, 2)
            k = self.k_proj(x).view(B, S, nkv, hd).transpose(1, 2)
            v = self.v_proj(x).view(B, S, nkv, hd).transpose(1, 2)
            cos, sin = rope(pos)
            q, k = apply_rotary(q, k, cos.to(q.dtype), sin.to(q.dtype))
            cache.update(layer, k, v, pos)
            qg = q.reshape(B, nkv, rep * S, hd)  # rows: (head within the group, token)
        if self._decode_fits(x, S, cache, kv_len, mask):
            from .. import _lib
            o = torch.empty((B, nh * hd), dtype=x.dtype, device=x.device)
            inv = float(np.float32(1.0) / np.float32(math.sqrt(hd)))
            _lib.call("hn_attn_decode", _lib.ptr(qg), _lib.ptr(cache.kt[layer]),
                      _lib.ptr(cache.v[layer]), cache.max_len, B, nkv, rep, hd, kv_len,
                      _lib.ptr(mask), inv, _lib.ptr(o), o.stride(0), _lib.stream(x.device))
            return self.o_proj(o.view(B, S, nh * hd))
        kt, vv = cache.get(layer, kv_len)
        scores = torch.matmul(qg, kt)  # [B, nkv, rep * S, kv_len]
        if x.is_cuda and kv_len <= 1024 and (mask is None or mask.dtype == torch.float16):
            p = attn_softmax(scores, mask, hd)
        else:
            scores = scores / math.sqrt(hd)
            if mask is not None:
                scores = (scores.view(B, nkv, rep, S, kv_len) + mask).view(B, nkv, rep * S,
                                                                           kv_len)
            p = F.softmax(scores, dim=-1, dtype=torch.float32).to(qg.dtype)
        o = torch.matmul(p, vv).view(B, nh, S, hd)
        return self.o_proj(o.transpose(1, 2).reshape(B, S, nh * hd))


def attn_softmax(scores: torch.Tensor, mask: Optional[torch.Tensor], head_dim: int) -> torch.Tensor:
    """fp16(softmax_fp32(fp16(scores / sqrt(head_dim)) + mask)) over the last
    dim (<= 1024), one launch (hn_attn_softmax): the torch formulation's
    rounding steps and reduction order.  scores [..., rows, L] fp16 with the
    mask's S rows fastest among the rows; mask [S, L] fp16 or None."""
    from .. import _lib
    L = scores.shape[-1]
    s2 = scores.reshape(-1, L)
    if s2.stride(-1) != 1 or s2.stride(0) < L:
        s2 = s2.contiguous()
    out = torch.empty((s2.shape[0], L), dtype=torch.float16, device=scores.device)
    # torch divides a Half tensor by a Python scalar as a multiply by the fp32
    # reciprocal of the fp32-rounded scalar
    inv = float(np.float32(1.0) / np.float32(math.sqrt(head_dim)))
    m2 = None
    if mask is not None:
        m2 = mask.reshape(-1, L)
        if m2.stride(-1) != 1:
            m2 = m2.contiguous()
    _lib.call("hn_attn_softmax", _lib.ptr(s2), s2.stride(0), _lib.ptr(m2),
              L if m2 is None else m2.stride(0), 1 if m2 is None else m2.shape[0], s2.shape[0],
              L, inv, _lib.ptr(out), L, _lib.stream(scores.device))
    return out.view(scores.shape)


def add_rmsnorm(x: torch.Tensor, res: Optional[torch.Tensor], norm: RMSNorm,
                gate: Optional[torch.Tensor] = None):
    """(x + res, norm(x + res)); res None: (x, norm(x)).  On the GPU one
    kernel (hn_add_rmsnorm) with the torch formulation's fp16 add and fp32
    normalisation.  gate: an fp16 router gate [E, H]; then a third result,
    the router logits [T, E] of the normalised rows (hn_add_rmsnorm_router)."""
    if not x.is_cuda:
        if res is not None:
            x = x + res
        h = norm(x)
        if gate is None:
            return x, h
        lg = F.linear(h, gate).float()
        return x, h, lg.reshape(-1, gate.shape[0])
    from .. import _lib
    H = x.shape[-1]
    assert norm.weight.dtype == torch.float16 and x.dtype == torch.float16
    x2 = x.reshape(-1, H).contiguous()
    T = x2.shape[0]
    out = torch.empty_like(x2)
    xo, r2 = x2, None
    if res is not None:
        r2 = res.reshape(-1, H).contiguous()
        xo = torch.empty_like(x2)
    if gate is None:
        _lib.call("hn_add_rmsnorm", _lib.ptr(x2), H, _lib.ptr(r2), H,
                  _lib.ptr(xo) if res is not None else None, H, _lib.ptr(norm.weight),
                  _lib.ptr(out), H, T, H, norm.eps, _lib.stream(x.device))
        return xo.view(x.shape), out.view(x.shape)
    assert gate.dtype == torch.float16 and gate.shape[1] == H and gate.stride(1) == 1
    E = gate.shape[0]
    lg = torch.empty((T, E), dtype=torch.float32, device=x.device)
    _lib.call("hn_add_rmsnorm_router", _lib.ptr(x2), H, _lib.ptr(r2), H,
              _lib.ptr(xo) if res is not None else None, H, _lib.ptr(norm.weight), _lib.ptr(out),
              H, T, H, norm.eps, _lib.ptr(gate), gate.stride(0), E, _lib.ptr(lg),
              _lib.stream(x.device))
    return xo.view(x.shape), out.view(x.shape), lg


def causal_mask(start: int, S: int, device, dtype=torch.float16) -> torch.Tensor:
    """[S, start + S]: token i (position start + i) sees positions <= start + i."""
    m = torch.full((S, start + S), float("-inf"), device=device, dtype=dtype)
    return torch.triu(m, diagonal=start + 1)


class DecoderBlock(nn.Module):
    def __init__(self, cfg: MixtralDecoderConfig, layer_idx: int, slots):
        super().__init__()
        self.layer_idx = layer_idx
        self.input_layernorm = RMSNorm(cfg.hidden_dim, cfg.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_dim, cfg.rms_norm_eps)
        self.self_attn = Attention(cfg)
        self.moe = MixtralMoELayer(cfg.hidden_dim, cfg.num_experts, cfg.experts_per_token,
                                   layer_idx=layer_idx, slots=slots)

    def forward(self, x, h, rope, pos, cache: KVCache, kv_len: int, mask, top_k: int,
                next_norm: "RMSNorm", fold: bool = True):
        """x + attn(h), then + moe(norm(.)) (model/mixtral.py:407-427), h =
        input_layernorm(x) given by the caller.  Returns (x after both
        residual adds, next_norm of it): the next block's input and its
        normalised rows.  fold: the MoE output's residual add and next_norm
        run inside the MoE block's last launch where it allows
        (forward_folded), else as one more launch."""
        a = self.self_attn(h, rope, pos, cache, self.layer_idx, kv_len, mask)
        T = h.shape[0] * h.shape[1]
        gw = self.moe.router.gate.weight
        lg = None
        if x.is_cuda and gw.dtype == torch.float16 and self.moe.takes_logits(T, top_k):
            # the router logits come out of the norm kernel (no gate product
            # in the routing launch)
            x, h, lg = add_rmsnorm(x, a, self.post_attention_layernorm, gate=gw)
        else:
            x, h = add_rmsnorm(x, a, self.post_attention_layernorm)
        if fold:
            r = self.moe.forward_folded(h, top_k, lg, x, next_norm.weight, next_norm.eps)
            if r is not None:
                return r
        m = self.moe(h, top_k=top_k, logits=lg) if lg is not None else self.moe(h, top_k=top_k)
        return add_rmsnorm(x, m, next_norm)


class MixtralDecoder(nn.Module):
    """Embeddings -> blocks -> norm -> LM head (model/mixtral.py:430-599), with
    every expert resident (one GpuExpertSlot per expert, `slots[layer][e]`).
    One RoPE table serves every layer (the positions are the same)."""

    def __init__(self, cfg: MixtralDecoderConfig, slots: List[list], device=None,
                 decode_top_k: int = 1):
        super().__init__()
        self.cfg = cfg
        self.decode_top_k = decode_top_k
        # the MoE block's residual add and the next RMSNorm inside its last
        # launch (hn_unpermute_add_rmsnorm) where the decode layer allows
        self.fold_moe_norm = True
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_dim)
        self.layers = nn.ModuleList([DecoderBlock(cfg, i, slots[i])
                                     for i in range(cfg.num_layers)])
        self.norm = RMSNorm(cfg.hidden_dim, cfg.rms_norm_eps)
        self.lm_head = nn.Linear(cfg.hidden_dim, cfg.vocab_size, bias=False)
        self.rotary = RotaryEmbedding(cfg.head_dim, cfg.max_position_embeddings, cfg.rope_theta,
                                      device)

    def new_cache(self, batch: int, max_len: int) -> KVCache:
        dev = self.embed_tokens.weight.device
        return KVCache(self.cfg.num_layers, batch, self.cfg.num_kv_heads, self.cfg.head_dim,
                       max_len, dev, self.embed_tokens.weight.dtype)

    def step(self, input_ids: torch.Tensor, pos: torch.Tensor, cache: KVCache, kv_len: int,
             mask: Optional[torch.Tensor], top_k: int) -> torch.Tensor:
        """One pass over every layer: tokens input_ids [B, S] at positions pos
        [S] (device int64), attention over the first kv_len cache positions.
        Does not move cache.cur_len."""
        x = self.embed_tokens(input_ids)
        x, h = add_rmsnorm(x, None, self.layers[0].input_layernorm)
        n = len(self.layers)
        for i, blk in enumerate(self.layers):
            nxt = self.layers[i + 1].input_layernorm if i + 1 < n else self.norm
            x, h = blk(x, h, self.rotary, pos, cache, kv_len, mask, top_k, nxt,
                       fold=self.fold_moe_norm)
        return self.lm_head(h)

    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor, cache: KVCache,
                top_k: Optional[int] = None) -> torch.Tensor:
        """input_ids [B, S] -> logits [B, S, vocab]; appends S positions to the
        cache (prefill when it is empty: top-2; decode: decode_top_k)."""
        B, S = input_ids.shape
        start = cache.cur_len
        if start + S > cache.max_len:
            raise RuntimeError(f"KV cache full ({start + S} > {cache.max_len})")
        if top_k is None:
            top_k = 2 if start == 0 else self.decode_top_k
        pos = torch.arange(start, start + S, device=input_ids.device)
        mask = causal_mask(start, S, input_ids.device) if S > 1 else None
        logits = self.step(input_ids, pos, cache, start + S, mask, top_k)
        cache.advance(S)
        return logits

    @torch.no_grad()
    def generate_greedy(self, input_ids: torch.Tensor, max_new_tokens: int,
                        cache: Optional[KVCache] = None, graph: bool = True) -> torch.Tensor:
        """Greedy (top-1 token) decode of max_new_tokens after the prompt; the
        batch shares one length (uniform prompts, no early stop).  graph: the
        decode steps are replayed from one captured HIP graph (GraphDecoder)."""
        B, S = input_ids.shape
        if cache is None:
            cache = self.new_cache(B, S + max_new_tokens)
        logits = self.forward(input_ids, cache)
        tok = logits[:, -1].argmax(-1, keepdim=True)
        out = [tok]
        if graph and max_new_tokens > 1:
            gd = GraphDecoder(self, cache, tok)
            for _ in range(max_new_tokens - 1):
                out.append(gd.step().clone())
            return torch.cat(out, dim=1)
        for _ in range(max_new_tokens - 1):
            tok = self.forward(tok, cache)[:, -1].argmax(-1, keepdim=True)
            out.append(tok)
        return torch.cat(out, dim=1)


class GraphDecoder:
    """Greedy decode steps replayed from captured HIP graphs.

    A captured step attends over the first L cache positions, L the current
    length rounded up to a multiple of `bucket` (positions past the current
    one masked to -inf, so they add exp(-inf) = 0 to the softmax); one graph
    per L the decode will reach, all captured up front into one memory pool.
    The step reads its position from a device scalar, writes the next tokens
    into a static buffer and advances the position itself: successive replays
    need no host work and no host-device sync.  `tok` holds the tokens fed to
    the next step; `logits` the last step's logits (valid until the next)."""

    def __init__(self, model: MixtralDecoder, cache: KVCache, tok: torch.Tensor,
                 bucket: int = 64):
        self.model, self.cache = model, cache
        dev = tok.device
        if cache.cur_len >= cache.max_len:
            raise RuntimeError(f"KV cache full ({cache.max_len} positions)")
        self.bucket = bucket
        self.tok = tok.clone()
        self.pos = torch.full((1,), cache.cur_len, dtype=torch.int64, device=dev)
        self.ar = torch.arange(cache.max_len, device=dev)
        self.graphs = {}  # L -> (graph, logits)
        self.logits = None
        tok0 = self.tok.clone()
        lens = sorted({self._len(n) for n in range(cache.cur_len, cache.max_len)})
        s = torch.cuda.Stream(device=dev)
        s.wait_stream(torch.cuda.current_stream(dev))
        with torch.no_grad(), torch.cuda.stream(s):
            self._body(lens[0])  # warm-up (allocator, library handles): rewritten below
        torch.cuda.current_stream(dev).wait_stream(s)
        self.pos.fill_(cache.cur_len)
        self.tok.copy_(tok0)
        pool = None
        for L in lens:  # capture runs nothing: the buffers keep their values
            g = torch.cuda.CUDAGraph()
            with torch.no_grad(), torch.cuda.graph(g, pool=pool):
                logits = self._body(L)
            pool = g.pool() if pool is None else pool
            self.graphs[L] = (g, logits)

    def _len(self, cur_len: int) -> int:
        """Cache positions a step at length cur_len attends over."""
        n = -(-(cur_len + 1) // self.bucket) * self.bucket
        return min(n, self.cache.max_len)

    def _body(self, L: int) -> torch.Tensor:
        mask = torch.zeros((1, L), dtype=torch.float16, device=self.tok.device).masked_fill_(
            self.ar[:L] > self.pos, float("-inf"))
        logits = self.model.step(self.tok, self.pos, self.cache, L, mask,
                                 self.model.decode_top_k)
        self.tok.copy_(logits[:, -1].argmax(-1, keepdim=True))
        self.pos.add_(1)
        return logits

    def step(self) -> torch.Tensor:
        """One decode step; returns the static buffer of the tokens it chose."""
        if self.cache.cur_len >= self.cache.max_len:
            raise RuntimeError(f"KV cache full ({self.cache.max_len} positions)")
        g, self.logits = self.graphs[self._len(self.cache.cur_len)]
        g.replay()
        self.cache.advance(1)
        return self.tok


def convert_dense_to_int4(model: nn.Module, group_size: int = 128) -> nn.Module:
    """The reference's INT4 option for non-expert weights (test_glm4_generate.py:
    262-280: convert_model_to_int4 with lm_head and the embeddings kept):
    every attention projection and dense MLP linear becomes an Int4Linear
    (kernels/int4_linear.py).  The MoE routers' gates stay fp16 (the routing
    kernels read them as such), as does the LM head."""
    from ..kernels.int4_linear import convert_model_to_int4
    return convert_model_to_int4(model, skip_layers=["lm_head", "embed", "router"],
                                 group_size=group_size)


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
    # the RoPE table is computed in fp32 (the cast to fp16 happens where it is applied)
    m.rotary = RotaryEmbedding(cfg.head_dim, cfg.max_position_embeddings, cfg.rope_theta, dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if name.endswith("norm.weight") or "layernorm" in name:
                p.fill_(1.0)
            else:
                p.copy_((torch.randn(p.shape, generator=g, device=dev) * 0.02).to(p.dtype))
    m.eval()
    return m

"""CPU checks of the decoder harness's attention and KV cache
(hydranet_amd/model/decoder.py), fp32: prefill of S tokens at once equals S
single-token decode steps through the cache (the causal mask's offset and the
cache's positions), grouped-query attention equals full multi-head attention
with each KV head repeated, and RoPE preserves norms and is relative
(q(m) . k(n) depends on m - n only)."""
import math

import torch

from hydranet_amd.model.decoder import (Attention, KVCache, MixtralDecoderConfig, RMSNorm,
                                        RotaryEmbedding, apply_rotary)


def _cfg():
    return MixtralDecoderConfig(num_layers=1, hidden_dim=64, intermediate_dim=128,
                                num_attention_heads=4, num_kv_heads=2, head_dim=16,
                                vocab_size=50, max_position_embeddings=32)


def test_prefill_equals_stepwise_decode():
    torch.manual_seed(0)
    cfg = _cfg()
    att = Attention(cfg).double()
    B, S = 2, 7
    x = torch.randn(B, S, cfg.hidden_dim, dtype=torch.float64)
    c1 = KVCache(1, B, cfg.num_kv_heads, cfg.head_dim, S, "cpu", torch.float64)
    pos = torch.arange(S).unsqueeze(0).expand(B, S)
    full = att(x, pos, c1, 0)
    c2 = KVCache(1, B, cfg.num_kv_heads, cfg.head_dim, S, "cpu", torch.float64)
    steps = []
    for t in range(S):
        steps.append(att(x[:, t:t + 1], pos[:, t:t + 1], c2, 0))
        c2.advance(1)
    torch.testing.assert_close(full, torch.cat(steps, 1), rtol=1e-10, atol=1e-10)
    # two-chunk prefill (the mask offset when the cache is not empty)
    c3 = KVCache(1, B, cfg.num_kv_heads, cfg.head_dim, S, "cpu", torch.float64)
    a = att(x[:, :3], pos[:, :3], c3, 0)
    c3.advance(3)
    b = att(x[:, 3:], pos[:, 3:], c3, 0)
    torch.testing.assert_close(full, torch.cat([a, b], 1), rtol=1e-10, atol=1e-10)


def test_gqa_equals_repeated_heads_mha():
    torch.manual_seed(1)
    cfg = _cfg()
    att = Attention(cfg).double()
    B, S, nh, nkv, hd = 1, 5, cfg.num_attention_heads, cfg.num_kv_heads, cfg.head_dim
    x = torch.randn(B, S, cfg.hidden_dim, dtype=torch.float64)
    cache = KVCache(1, B, nkv, hd, S, "cpu", torch.float64)
    pos = torch.arange(S).unsqueeze(0)
    got = att(x, pos, cache, 0)
    # textbook causal attention, written out per head
    q = (x @ att.q_proj.weight.T).view(B, S, nh, hd).transpose(1, 2)
    k = (x @ att.k_proj.weight.T).view(B, S, nkv, hd).transpose(1, 2)
    v = (x @ att.v_proj.weight.T).view(B, S, nkv, hd).transpose(1, 2)
    cos, sin = att.rope(pos)
    q, k = apply_rotary(q, k, cos.double(), sin.double())
    o = torch.zeros(B, nh, S, hd, dtype=torch.float64)
    for h in range(nh):
        kh, vh = k[:, h * nkv // nh], v[:, h * nkv // nh]
        for i in range(S):
            sc = (q[:, h, i:i + 1] @ kh[:, :i + 1].transpose(1, 2)) / math.sqrt(hd)
            o[:, h, i] = (torch.softmax(sc, -1) @ vh[:, :i + 1])[:, 0]
    ref = o.transpose(1, 2).reshape(B, S, nh * hd) @ att.o_proj.weight.T
    # the module's softmax runs in fp32 (as the reference's): fp32-level agreement
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-6)


def test_rope_norm_and_relative_position():
    rope = RotaryEmbedding(16, 64, 1e6)
    torch.manual_seed(2)
    q = torch.randn(1, 1, 1, 16, dtype=torch.float64)
    k = torch.randn(1, 1, 1, 16, dtype=torch.float64)

    def rot(v, p):
        c, s = rope(torch.tensor([[p]]))
        return apply_rotary(v, v, c.double(), s.double())[0]

    for p in (0, 5, 40):
        torch.testing.assert_close(rot(q, p).norm(), q.norm(), rtol=1e-6, atol=1e-6)
    d1 = (rot(q, 10) * rot(k, 7)).sum()
    d2 = (rot(q, 33) * rot(k, 30)).sum()
    torch.testing.assert_close(d1, d2, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(rot(q, 0), q)


def test_rmsnorm_matches_definition():
    n = RMSNorm(8, 1e-5)
    with torch.no_grad():
        n.weight.copy_(torch.arange(1, 9, dtype=torch.float32))
    x = torch.randn(3, 8).half()
    ref = (x.float() / torch.sqrt(x.float().pow(2).mean(-1, keepdim=True) + 1e-5)
           * torch.arange(1, 9)).half()
    torch.testing.assert_close(n(x), ref, rtol=0, atol=0)

"""CPU checks of the decoder harness's attention and KV cache
(hydranet_amd/model/decoder.py), float64: prefill of S tokens at once equals S
single-token decode steps through the cache (the causal mask's offset and the
cache's positions), attention over the whole cache with the later positions
masked equals attention over the filled part (the captured decode step's
form), grouped-query attention equals textbook per-head attention with KV head
h // (heads / kv_heads), and RoPE preserves norms and is relative
(q(m) . k(n) depends on m - n only)."""
import math

import torch

from hydranet_amd.model.decoder import (Attention, KVCache, MixtralDecoderConfig, RMSNorm,
                                        RotaryEmbedding, apply_rotary, causal_mask)


def _cfg():
    return MixtralDecoderConfig(num_layers=1, hidden_dim=64, intermediate_dim=128,
                                num_attention_heads=4, num_kv_heads=2, head_dim=16,
                                vocab_size=50, max_position_embeddings=32)


def _setup(seed):
    torch.manual_seed(seed)
    cfg = _cfg()
    att = Attention(cfg).double()
    rope = RotaryEmbedding(cfg.head_dim, 32, cfg.rope_theta).double()
    return cfg, att, rope


def _run(att, rope, x, cache, start, mask=None, kv_len=None):
    S = x.shape[1]
    pos = torch.arange(start, start + S)
    if mask is None and S > 1:
        mask = causal_mask(start, S, "cpu", torch.float64)
    return att(x, rope, pos, cache, 0, kv_len or start + S, mask)


def test_prefill_equals_stepwise_decode():
    cfg, att, rope = _setup(0)
    B, S = 2, 7
    x = torch.randn(B, S, cfg.hidden_dim, dtype=torch.float64)
    mk = lambda L: KVCache(1, B, cfg.num_kv_heads, cfg.head_dim, L, "cpu", torch.float64)
    c1 = mk(S)
    full = _run(att, rope, x, c1, 0)
    c2 = mk(S)
    steps = [_run(att, rope, x[:, t:t + 1], c2, t) for t in range(S)]
    # the module's softmax runs in fp32 (as the reference's): fp32-level agreement
    torch.testing.assert_close(full, torch.cat(steps, 1), rtol=1e-5, atol=1e-7)
    # two-chunk prefill (the mask offset when the cache is not empty)
    c3 = mk(S)
    a = _run(att, rope, x[:, :3], c3, 0)
    b = _run(att, rope, x[:, 3:], c3, 3)
    torch.testing.assert_close(full, torch.cat([a, b], 1), rtol=1e-5, atol=1e-7)
    # decode over the whole cache with the positions after the current one masked
    L = 12
    c4 = mk(L)
    ar = torch.arange(L)
    outs = []
    for t in range(S):
        m = torch.zeros(1, L, dtype=torch.float64).masked_fill_(ar > t, float("-inf"))
        outs.append(_run(att, rope, x[:, t:t + 1], c4, t, mask=m, kv_len=L))
    torch.testing.assert_close(full, torch.cat(outs, 1), rtol=1e-5, atol=1e-7)


def test_gqa_equals_textbook_attention():
    cfg, att, rope = _setup(1)
    B, S, nh, nkv, hd = 2, 5, cfg.num_attention_heads, cfg.num_kv_heads, cfg.head_dim
    x = torch.randn(B, S, cfg.hidden_dim, dtype=torch.float64)
    cache = KVCache(1, B, nkv, hd, S, "cpu", torch.float64)
    got = _run(att, rope, x, cache, 0)
    q = (x @ att.q_proj.weight.T).view(B, S, nh, hd).transpose(1, 2)
    k = (x @ att.k_proj.weight.T).view(B, S, nkv, hd).transpose(1, 2)
    v = (x @ att.v_proj.weight.T).view(B, S, nkv, hd).transpose(1, 2)
    cos, sin = rope(torch.arange(S))
    q, k = apply_rotary(q, k, cos, sin)
    o = torch.zeros(B, nh, S, hd, dtype=torch.float64)
    for h in range(nh):
        kh, vh = k[:, h // (nh // nkv)], v[:, h // (nh // nkv)]
        for i in range(S):
            sc = (q[:, h, i:i + 1] @ kh[:, :i + 1].transpose(1, 2)) / math.sqrt(hd)
            o[:, h, i] = (torch.softmax(sc, -1) @ vh[:, :i + 1])[:, 0]
    ref = o.transpose(1, 2).reshape(B, S, nh * hd) @ att.o_proj.weight.T
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-6)
    # the cache holds the rotated keys (transposed) and the values
    torch.testing.assert_close(cache.kt[0][..., :S], k.transpose(2, 3))
    torch.testing.assert_close(cache.v[0][:, :, :S], v)


def test_rope_norm_and_relative_position():
    rope = RotaryEmbedding(16, 64, 1e6)
    torch.manual_seed(2)
    q = torch.randn(1, 1, 1, 16, dtype=torch.float64)
    k = torch.randn(1, 1, 1, 16, dtype=torch.float64)

    def rot(v, p):
        c, s = rope(torch.tensor([p]))
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


def test_causal_mask_brute_force():
    for start, S in [(0, 1), (0, 5), (3, 4), (7, 1)]:
        m = causal_mask(start, S, "cpu", torch.float32)
        assert m.shape == (S, start + S)
        for i in range(S):
            for j in range(start + S):
                want = 0.0 if j <= start + i else float("-inf")
                assert m[i, j].item() == want, (start, S, i, j)


def test_kv_cache_bounds():
    c = KVCache(1, 1, 1, 4, 3, "cpu", torch.float32)
    c.advance(3)
    try:
        c.advance(1)
    except AssertionError:
        pass
    else:
        raise AssertionError("advance past max_len must fail")

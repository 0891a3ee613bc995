"""GPU tests of the decoder-step kernels (hn_add_rmsnorm, hn_rope_append)
against the reference's torch formulation of the same steps
(model/mixtral.py:23-37 RMSNorm, 82-101 RoPE; the KV-cache append):
the residual add, RoPE and the cache writes bit for bit; RMSNorm within one
fp16 ulp (fp32 mean in another summation order), nearly all elements equal."""
import numpy as np
import pytest
import torch

from hydranet_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _torch_rmsnorm(x, w, eps):
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (w * xf).to(torch.float16)


@pytest.mark.parametrize("T,H", [(1, 4096), (64, 4096), (5, 512), (3, 8192), (0, 4096)])
def test_add_rmsnorm(T, H):
    g = torch.Generator(device=DEV).manual_seed(T * 7 + H)
    x = torch.randn(T, H, generator=g, device=DEV).half()
    r = (torch.randn(T, H, generator=g, device=DEV) * 0.5).half()
    w = (1 + 0.1 * torch.randn(H, generator=g, device=DEV)).half()
    st = _lib.stream()
    for res in (None, r):
        out = torch.empty_like(x)
        xo = torch.empty_like(x)
        _lib.call("hn_add_rmsnorm", _lib.ptr(x), H, _lib.ptr(res), H,
                  _lib.ptr(xo) if res is not None else None, H, _lib.ptr(w), _lib.ptr(out), H,
                  T, H, 1e-5, st)
        xs = x if res is None else x + res
        if res is not None:
            assert torch.equal(xo, xs)
        ref = _torch_rmsnorm(xs, w, 1e-5)
        if T == 0:
            continue
        ulp = torch.pow(2.0, torch.floor(torch.log2(ref.float().abs().clamp_min(2.0 ** -14))) - 10)
        assert bool(((out.float() - ref.float()).abs() <= ulp).all())
        assert (out != ref).float().mean().item() < 0.02


@pytest.mark.parametrize("T,H,E", [(1, 4096, 8), (64, 4096, 8), (5, 512, 16), (3, 1024, 3)])
def test_add_rmsnorm_router(T, H, E):
    """The norm output equals hn_add_rmsnorm's bit for bit; the logits are the
    fp16 gate product of that output: fp16 values within one fp16 ulp of the
    float64 product rounded to fp16 (the fp32 sum's order is the kernel's)."""
    g = torch.Generator(device=DEV).manual_seed(T * 31 + E)
    x = torch.randn(T, H, generator=g, device=DEV).half()
    r = (torch.randn(T, H, generator=g, device=DEV) * 0.5).half()
    w = (1 + 0.1 * torch.randn(H, generator=g, device=DEV)).half()
    gate = (torch.randn(E, H, generator=g, device=DEV) * 0.02).half()
    st = _lib.stream()
    out0, xo0 = torch.empty_like(x), torch.empty_like(x)
    _lib.call("hn_add_rmsnorm", _lib.ptr(x), H, _lib.ptr(r), H, _lib.ptr(xo0), H, _lib.ptr(w),
              _lib.ptr(out0), H, T, H, 1e-5, st)
    out1, xo1 = torch.empty_like(x), torch.empty_like(x)
    lg = torch.full((T, E), float("nan"), device=DEV)
    _lib.call("hn_add_rmsnorm_router", _lib.ptr(x), H, _lib.ptr(r), H, _lib.ptr(xo1), H,
              _lib.ptr(w), _lib.ptr(out1), H, T, H, 1e-5, _lib.ptr(gate), H, E, _lib.ptr(lg), st)
    torch.cuda.synchronize()
    assert torch.equal(out1, out0) and torch.equal(xo1, xo0)
    assert torch.equal(lg, lg.half().float()), "logits hold fp16 values"
    ref = (out0.double().cpu() @ gate.double().cpu().t()).half().double()
    ulp = torch.pow(2.0, torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -14))) - 10)
    assert bool(((lg.double().cpu() - ref).abs() <= ulp).all())


def test_add_rmsnorm_router_rejects_bad_arguments():
    x = torch.zeros(2, 512, device=DEV).half()
    w = torch.ones(512, device=DEV).half()
    gate = torch.zeros(17, 512, device=DEV).half()
    lg = torch.zeros(2, 17, device=DEV)
    with pytest.raises(RuntimeError, match="E <= 16"):
        _lib.call("hn_add_rmsnorm_router", _lib.ptr(x), 512, None, 512, None, 512, _lib.ptr(w),
                  _lib.ptr(x), 512, 2, 512, 1e-5, _lib.ptr(gate), 512, 17, _lib.ptr(lg),
                  _lib.stream())


def test_add_rmsnorm_in_place_residual():
    """x_out may alias x (the residual stream updated in place)."""
    H, T = 1024, 4
    x = torch.randn(T, H, device=DEV).half()
    r = torch.randn(T, H, device=DEV).half()
    w = torch.ones(H, device=DEV).half()
    want = x + r
    out = torch.empty_like(x)
    _lib.call("hn_add_rmsnorm", _lib.ptr(x), H, _lib.ptr(r), H, _lib.ptr(x), H, _lib.ptr(w),
              _lib.ptr(out), H, T, H, 1e-5, _lib.stream())
    assert torch.equal(x, want)


@pytest.mark.parametrize("rows,L,S", [(2048, 576, 1), (64, 1, 1), (128, 7, 1), (256, 64, 1),
                                      (256, 65, 1), (512, 1000, 1), (96, 1024, 1),
                                      (4 * 2 * 12, 12, 12), (2 * 4 * 40, 200, 40)])
@pytest.mark.parametrize("masked", [False, True])
def test_attn_softmax_matches_torch_formulation(rows, L, S, masked):
    """hn_attn_softmax against the reference's steps run by torch on the same
    GPU (scores / sqrt(head_dim), + mask, F.softmax(dtype=float32), .to(fp16)):
    bit for bit.  Masks: the decode graph's tail of -inf (S = 1) or a causal
    mask (S > 1); one row of large scores exercises the max subtraction."""
    import math
    from hydranet_amd.model.decoder import attn_softmax, causal_mask
    g = torch.Generator(device=DEV).manual_seed(rows + L)
    sc = (torch.randn(rows // S, S, L, generator=g, device=DEV) * 6).half()
    sc[0, 0, : min(L, 5)] = 300.0
    mask = None
    if masked:
        if S == 1:
            mask = torch.zeros((1, L), dtype=torch.float16, device=DEV)
            mask[:, L - L // 5:] = float("-inf") if L > 1 else 0.0
        else:
            mask = causal_mask(L - S, S, DEV)
    got = attn_softmax(sc, mask, 128)
    ref = sc / math.sqrt(128)
    if mask is not None:
        ref = ref + mask
    ref = torch.softmax(ref, dim=-1, dtype=torch.float32).to(torch.float16)
    torch.cuda.synchronize()
    diff = (got != ref)
    assert not bool(diff.any()), (int(diff.sum()), float((got.float() - ref.float()).abs().max()))


@pytest.mark.parametrize("B,nkv,rep,L,max_len,masked", [
    (2, 2, 4, 1, 8, False), (3, 2, 4, 7, 16, True), (2, 8, 4, 512, 768, False),
    (4, 8, 4, 640, 768, True), (2, 2, 2, 777, 784, False), (2, 2, 1, 1024, 1024, True),
    (1, 1, 4, 300, 304, False), (64, 8, 4, 576, 768, True)])
def test_attn_decode_vs_two_products(B, nkv, rep, L, max_len, masked):
    """hn_attn_decode (one launch) against the reference's steps run by torch
    on the same GPU: fp16 score product, / sqrt(head_dim), + mask,
    F.softmax(dtype=float32).to(fp16), fp16 value product; and against a
    float64 CPU evaluation of the same roundings.  fp16 outputs within
    max-abs 1e-2 and relative 2e-3 of both (the fp32 sums run in another
    order than the library GEMM's).  Cache positions past L hold NaN, which
    must not reach the result."""
    import math
    from hydranet_amd.model.decoder import attn_softmax
    hd = 128
    print(f"[attn_decode] B={B} nkv={nkv} rep={rep} L={L} max_len={max_len} masked={masked}",
          flush=True)
    g = torch.Generator(device=DEV).manual_seed(B * 1000 + L)
    q = torch.randn(B, nkv, rep, hd, generator=g, device=DEV).half()
    kt = torch.randn(B, nkv, hd, max_len, generator=g, device=DEV).half()
    v = torch.randn(B, nkv, max_len, hd, generator=g, device=DEV).half()
    kt[..., L:] = float("nan")
    v[:, :, L:] = float("nan")
    mask = None
    if masked:
        mask = torch.zeros((1, L), dtype=torch.float16, device=DEV)
        mask[:, L - L // 4:] = float("-inf") if L > 1 else 0.0
    out = torch.full((B, nkv * rep * hd), float("nan"), dtype=torch.float16, device=DEV)
    inv = float(np.float32(1.0) / np.float32(math.sqrt(hd)))
    _lib.call("hn_attn_decode", _lib.ptr(q), _lib.ptr(kt), _lib.ptr(v), max_len, B, nkv, rep,
              hd, L, _lib.ptr(mask), inv, _lib.ptr(out), out.stride(0), _lib.stream())
    # the reference's two products with the softmax between them
    sc = torch.matmul(q, kt[..., :L].contiguous())
    p = attn_softmax(sc, mask, hd)
    ref = torch.matmul(p, v[:, :, :L].contiguous()).reshape(B, -1)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    err = (out.float() - ref.float()).abs()
    assert bool((err <= 1e-2 + 2e-3 * ref.float().abs()).all()), float(err.max())
    # float64 on the CPU with the same fp16 roundings
    qd, kd, vd = q.double().cpu(), kt[..., :L].double().cpu(), v[:, :, :L].double().cpu()
    s16 = (qd @ kd).half()
    a = (s16.float() * inv).half()
    if mask is not None:
        a = (a.float() + mask.float().cpu()).half()
    p64 = torch.softmax(a.double(), dim=-1).half()
    ref64 = (p64.double() @ vd).reshape(B, -1)
    err = (out.double().cpu() - ref64).abs()
    assert bool((err <= 1e-2 + 2e-3 * ref64.abs()).all()), float(err.max())


@pytest.mark.parametrize("B,nkv,rep,max_len,p,L,masked", [
    (3, 2, 4, 64, 20, 21, False), (2, 8, 4, 768, 600, 640, True), (2, 2, 2, 16, 15, 16, False),
    (1, 1, 1, 8, 0, 1, False), (64, 8, 4, 768, 513, 576, True)])
def test_attn_decode_rope_equals_rope_append_then_attention(B, nkv, rep, max_len, p, L, masked):
    """hn_attn_decode_rope (RoPE, cache append and attention in one launch)
    against hn_rope_append followed by hn_attn_decode on copies of the same
    caches: the outputs and both caches bit for bit (the new key and value
    at position p, everything else untouched)."""
    import math
    hd = 128
    nh = nkv * rep
    print(f"[attn_decode_rope] B={B} nkv={nkv} rep={rep} max_len={max_len} p={p} L={L}",
          flush=True)
    g = torch.Generator(device=DEV).manual_seed(B * 7 + p)
    qkv = torch.randn(B, (nh + 2 * nkv) * hd, generator=g, device=DEV).half()
    kt = torch.randn(B, nkv, hd, max_len, generator=g, device=DEV).half()
    v = torch.randn(B, nkv, max_len, hd, generator=g, device=DEV).half()
    npos = max(max_len, 1024)
    inv_f = 1.0 / (1e6 ** (torch.arange(0, hd, 2, device=DEV).float() / hd))
    t = torch.arange(npos, device=DEV, dtype=torch.float32)
    emb = torch.cat([torch.outer(t, inv_f)] * 2, dim=-1)
    cos_t, sin_t = emb.cos().contiguous(), emb.sin().contiguous()
    pos = torch.tensor([p], dtype=torch.int64, device=DEV)
    mask = None
    if masked:
        mask = torch.zeros((1, L), dtype=torch.float16, device=DEV)
        mask[:, p + 1:] = float("-inf")
    inv = float(np.float32(1.0) / np.float32(math.sqrt(hd)))
    st = _lib.stream()
    # separate launches on copies
    kt_a, v_a = kt.clone(), v.clone()
    qg = torch.empty(B, nkv, rep, hd, dtype=torch.float16, device=DEV)
    ld = qkv.stride(0)
    base = qkv.data_ptr()
    _lib.call("hn_rope_append", base, ld, base + 2 * nh * hd, ld, base + 2 * (nh + nkv) * hd, ld,
              _lib.ptr(cos_t), _lib.ptr(sin_t), _lib.ptr(pos), B, 1, nh, nkv, hd, _lib.ptr(qg),
              _lib.ptr(kt_a), _lib.ptr(v_a), max_len, st)
    out_a = torch.empty(B, nh * hd, dtype=torch.float16, device=DEV)
    _lib.call("hn_attn_decode", _lib.ptr(qg), _lib.ptr(kt_a), _lib.ptr(v_a), max_len, B, nkv, rep,
              hd, L, _lib.ptr(mask), inv, _lib.ptr(out_a), out_a.stride(0), st)
    # one launch
    kt_b, v_b = kt.clone(), v.clone()
    out_b = torch.full((B, nh * hd), float("nan"), dtype=torch.float16, device=DEV)
    _lib.call("hn_attn_decode_rope", _lib.ptr(qkv), ld, _lib.ptr(cos_t), _lib.ptr(sin_t),
              _lib.ptr(pos), _lib.ptr(kt_b), _lib.ptr(v_b), max_len, B, nkv, rep, hd, L,
              _lib.ptr(mask), inv, _lib.ptr(out_b), out_b.stride(0), st)
    torch.cuda.synchronize()
    assert torch.equal(kt_a, kt_b) and torch.equal(v_a, v_b)
    assert not torch.equal(kt_a[..., p], kt[..., p])  # the step's key was written
    assert torch.isfinite(out_b).all()
    assert torch.equal(out_a, out_b)


def test_attn_decode_rejects_bad_shapes():
    for args in ((64, 1, 1, 4, 96, 8), (64, 1, 1, 3, 128, 8), (64, 1, 1, 4, 128, 1025),
                 (60, 1, 1, 4, 128, 8), (8, 1, 1, 4, 128, 9)):
        max_len, B, nkv, rep, hd, L = args
        with pytest.raises(RuntimeError, match="hn_attn_decode"):
            _lib.call("hn_attn_decode", None, None, None, max_len, B, nkv, rep, hd, L, None,
                      0.1, None, 4096, None)


def _rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


@pytest.mark.parametrize("B,S,start", [(3, 1, 7), (2, 5, 0), (2, 4, 9), (64, 1, 600)])
def test_rope_append(B, S, start):
    nh, nkv, hd, L = 8, 2, 64, 1024
    rep = nh // nkv
    g = torch.Generator(device=DEV).manual_seed(B * 100 + S)
    q = torch.randn(B * S, nh * hd, generator=g, device=DEV).half()
    k = torch.randn(B * S, nkv * hd, generator=g, device=DEV).half()
    v = torch.randn(B * S, nkv * hd, generator=g, device=DEV).half()
    inv = 1.0 / (1e6 ** (torch.arange(0, hd, 2, device=DEV).float() / hd))
    t = torch.arange(L, device=DEV, dtype=torch.float32)
    emb = torch.cat([torch.outer(t, inv)] * 2, -1)
    cos_t, sin_t = emb.cos().contiguous(), emb.sin().contiguous()
    pos = torch.arange(start, start + S, device=DEV)
    qg = torch.full((B, nkv, rep * S, hd), 7.0, dtype=torch.float16, device=DEV)
    kt = torch.zeros(B, nkv, hd, L, dtype=torch.float16, device=DEV)
    vc = torch.zeros(B, nkv, L, hd, dtype=torch.float16, device=DEV)
    _lib.call("hn_rope_append", _lib.ptr(q), nh * hd, _lib.ptr(k), nkv * hd, _lib.ptr(v),
              nkv * hd, _lib.ptr(cos_t), _lib.ptr(sin_t), _lib.ptr(pos), B, S, nh, nkv, hd,
              _lib.ptr(qg), _lib.ptr(kt), _lib.ptr(vc), L, _lib.stream())
    # torch formulation: fp16 tables, fp16 products and sum
    c, s = cos_t[pos].half(), sin_t[pos].half()
    qh = q.view(B, S, nh, hd).transpose(1, 2)
    kh = k.view(B, S, nkv, hd).transpose(1, 2)
    vh = v.view(B, S, nkv, hd).transpose(1, 2)
    q_ref = qh * c + _rotate_half(qh) * s
    k_ref = kh * c + _rotate_half(kh) * s
    assert torch.equal(qg, q_ref.reshape(B, nkv, rep * S, hd))
    kt_ref = torch.zeros_like(kt)
    kt_ref[..., start:start + S] = k_ref.transpose(2, 3)
    vc_ref = torch.zeros_like(vc)
    vc_ref[:, :, start:start + S] = vh
    assert torch.equal(kt, kt_ref)
    assert torch.equal(vc, vc_ref)

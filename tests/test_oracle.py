"""CPU tests pinning the oracle (oracle/) before it is trusted as the checker.

Each oracle function is checked against something it did not produce:
  * golden vectors written by the reference's own code (tests/golden/),
  * closed forms checked exhaustively (dequant over every nibble x every fp16 scale),
  * invariants from the reference's tests, and brute force on tiny inputs.
A planted-mistake test shows the golden checks catch a plausible slip.
"""
import json
import os

import numpy as np
import pytest
import torch

import oracle
from oracle import torch_ref

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _npz(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def _f16(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16)


# --------------------------------------------------------------------------- packer
def _quantize_cases():
    z = _npz("quantize_tensor.npz")
    names = sorted({k.split("/")[0] for k in z.files})
    return z, names


def test_quantize_tensor_matches_reference_golden():
    z, names = _quantize_cases()
    assert len(names) >= 5
    for n in names:
        w = _f16(z[f"{n}/w"])
        g = int(z[f"{n}/group"])
        packed, scales = oracle.quantize(w, g, mode=0)
        np.testing.assert_array_equal(packed, z[f"{n}/packed"], err_msg=n)
        np.testing.assert_array_equal(scales.view(np.uint16), z[f"{n}/scales"], err_msg=n)


def test_dequantize_matches_reference_golden():
    z, names = _quantize_cases()
    for n in names:
        g = int(z[f"{n}/group"])
        deq = oracle.dequant(z[f"{n}/packed"], _f16(z[f"{n}/scales"]), g)
        np.testing.assert_array_equal(deq.view(np.uint16), z[f"{n}/dequant"], err_msg=n)


def test_quantize_weight_int4linear_matches_reference_golden():
    z = np.load(os.path.join(GOLD, "quantize_weight.npz"), allow_pickle=False)
    keys = sorted({k.split("/")[0] for k in z.files})
    assert len(keys) == 6
    for key in keys:
        gs = int(key.split("_g")[1])
        w = z[f"{key}/w"]
        w = _f16(w) if key.startswith("f16") else w.astype(np.float32)
        packed, scales = oracle.quantize(w, gs, mode=1)
        np.testing.assert_array_equal(packed, z[f"{key}/packed"], err_msg=key)
        np.testing.assert_array_equal(scales.view(np.uint16), z[f"{key}/scales"], err_msg=key)


def test_planted_nibble_order_mistake_is_caught():
    # a packer that swapped nibble order must fail the golden comparison
    z, names = _quantize_cases()
    n = names[0]
    packed, _ = oracle.quantize(_f16(z[f"{n}/w"]), int(z[f"{n}/group"]), mode=0)
    swapped = ((packed >> 4) | (packed << 4)).astype(np.uint8)
    assert not np.array_equal(swapped, z[f"{n}/packed"])


def test_dequant_closed_form_exhaustive():
    # every nibble x every finite fp16 scale: fp16((n - 8) * s), numpy's fp16
    # multiply rounds the exact product once
    s_bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    s = s_bits.view(np.float16)
    s = s[np.isfinite(s)]
    K = 32
    rows = s.size
    nib = np.arange(16, dtype=np.uint8)
    codes = np.tile(nib, K // 16)  # k = 0..31 -> nibble k % 16
    packed_row = (codes[1::2] << 4) | codes[0::2]
    packed = np.tile(packed_row, (rows, 1)).astype(np.uint8)
    scales = s.reshape(rows, 1)
    got = oracle.dequant(packed, scales, K)
    with np.errstate(over="ignore"):
        exp = (codes.astype(np.float16)[None, :] - np.float16(8)) * scales
    np.testing.assert_array_equal(got.view(np.uint16), exp.astype(np.float16).view(np.uint16))


def test_quantize_invariants_random():
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((64, 512)) * 0.02).astype(np.float16)
    packed, scales = oracle.quantize(w, 128, mode=0)
    lo, hi = packed & 0xF, packed >> 4
    assert lo.min() >= 1 and hi.min() >= 1  # |w/s| <= 7(1+2^-11)^2 -> q in [-7, 7]
    deq = oracle.dequant(packed, scales, 128).astype(np.float32)
    s = np.repeat(scales.astype(np.float32), 128, axis=1)
    # |deq - w| <= s/2 plus fp16 rounding slack
    assert np.all(np.abs(deq - w.astype(np.float32)) <= s * 0.5 + s * 2e-3 + 1e-7)
    # reference test_int4_pack.py:65-66 error bounds
    assert np.abs(deq - w).max() < 0.1 and np.abs(deq - w).mean() < 0.01


# --------------------------------------------------------------------------- expert MLP
def test_torch_ref_expert_mlp_matches_reference_golden():
    z = _npz("expert_mlp.npz")
    H, I, gs = (int(v) for v in z["dims"])
    t = {k: torch.from_numpy(z[k]) for k in ("gate_packed", "up_packed", "down_packed")}
    for k in ("gate_scales", "up_scales", "down_scales", "x", "y"):
        t[k] = torch.from_numpy(_f16(z[k]).copy())
    y = torch_ref.expert_mlp(t["x"], t["gate_packed"], t["gate_scales"], t["up_packed"],
                             t["up_scales"], t["down_packed"], t["down_scales"], gs)
    assert torch.equal(y.view(torch.int16), t["y"].view(torch.int16))


def test_c_int4_linear_agrees_with_torch_dequant_matmul():
    rng = np.random.default_rng(7)
    N, K, M, g = 48, 256, 3, 128
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
    x = rng.standard_normal((M, K)).astype(np.float16)
    packed, scales = oracle.quantize(w, g)
    got = oracle.int4_linear(x, packed, scales, g).astype(np.float32)
    deq = oracle.dequant(packed, scales, g).astype(np.float64)
    exp = x.astype(np.float64) @ deq.T
    np.testing.assert_allclose(got, exp, rtol=2e-3, atol=2e-3)


# --------------------------------------------------------------------------- routers
def test_topk_router_matches_reference_golden_including_ties():
    z = _npz("topk_router.npz")
    h = _f16(z["h"]).reshape(-1, 256)
    gate = _f16(z["gate"])
    for k in (1, 2):
        logits_ref = z[f"k{k}/logits"].reshape(-1, 8)
        idx, w = oracle.router_topk(logits_ref, k, mode=0)
        ref_idx = z[f"k{k}/idx"].reshape(-1, k)
        # torch's CPU topk orders equal values by its nth_element pass (unspecified);
        # tie-free rows must match exactly, tied rows must select the same values
        srt = -np.sort(-logits_ref, axis=1)
        tie_free = srt[:, k - 1] != srt[:, k]
        assert tie_free.sum() >= logits_ref.shape[0] - 4
        np.testing.assert_array_equal(idx[tie_free], ref_idx[tie_free])
        np.testing.assert_array_equal(np.take_along_axis(logits_ref, idx, 1),
                                      np.take_along_axis(logits_ref, ref_idx, 1))
        wr = _f16(z[f"k{k}/w"]).reshape(-1, k).astype(np.float32)
        np.testing.assert_allclose(w.astype(np.float32), wr, atol=1e-3, rtol=0)
        # reference invariant (tests/test_model_math.py:151-153)
        np.testing.assert_allclose(w.astype(np.float32).sum(-1), 1.0, atol=2e-3)
    # C logits (fp16-rounded fp32 sum) vs the reference's fp16 Linear
    lg = oracle.router_logits(h, gate)
    np.testing.assert_allclose(lg, z["k2/logits"].reshape(-1, 8), atol=2e-3, rtol=2e-3)


def test_sigmoid_router_matches_reference_golden():
    z = _npz("sigmoid_router.npz")
    E, k = int(z["cfg"][0]), int(z["cfg"][1])
    h = _f16(z["h"]).reshape(-1, 256)
    w = z["w"].astype(np.float32)
    logits_t = torch.nn.functional.linear(torch.from_numpy(h.astype(np.float32)),
                                          torch.from_numpy(w)).numpy()
    idx, wt = oracle.router_topk(logits_t, k, mode=1, scaling=float(z["scaling"]))
    np.testing.assert_array_equal(idx, z["idx"])
    np.testing.assert_allclose(wt.astype(np.float32), _f16(z["wts"]).astype(np.float32),
                               atol=1e-3, rtol=0)
    lg = oracle.router_logits(h, w)
    np.testing.assert_allclose(lg, logits_t, atol=1e-4, rtol=1e-4)


def _grouped_cases():
    z = _npz("grouped_router.npz")
    names = sorted({k.split("/")[0] for k in z.keys()})
    return z, names


def test_grouped_router_matches_reference_golden():
    """torch_ref.glm_router with group-limited selection and norm_topk_prob=False
    equals GLM4SigmoidRouter.forward run by the reference (model/glm4.py:285-307),
    indices and fp16 weights bit for bit."""
    z, names = _grouped_cases()
    assert len(names) == 4
    for nm in names:
        E, k, ng, tg, norm = (int(v) for v in z[f"{nm}/cfg"])
        h = torch.from_numpy(_f16(z[f"{nm}/h"]).reshape(-1, 256))
        w = torch.from_numpy(z[f"{nm}/w"])
        idx, wt, _ = torch_ref.glm_router(h, w, k, scaling=float(z[f"{nm}/scaling"]),
                                          n_group=ng, topk_group=tg, norm_topk_prob=bool(norm))
        np.testing.assert_array_equal(idx.numpy(), z[f"{nm}/idx"], err_msg=nm)
        np.testing.assert_array_equal(wt.numpy().view(np.uint16), z[f"{nm}/wts"], err_msg=nm)


def test_c_oracle_grouped_router_matches_reference_golden():
    """The C oracle's group limit + sigmoid top-k (modes 1 and 2) over fp32
    logits reproduces the reference's grouped / unnormalised routing."""
    z, names = _grouped_cases()
    for nm in names:
        E, k, ng, tg, norm = (int(v) for v in z[f"{nm}/cfg"])
        h = _f16(z[f"{nm}/h"]).reshape(-1, 256).astype(np.float32)
        lg = torch.nn.functional.linear(torch.from_numpy(h),
                                        torch.from_numpy(z[f"{nm}/w"])).numpy()
        sel = oracle.router_group_limit(lg, ng, tg) if ng > 1 else lg
        if ng > 1:
            assert (np.isinf(sel).reshape(len(lg), ng, -1).all(-1).sum(-1) == ng - tg).all()
        idx, wt = oracle.router_topk(sel, k, mode=1 if norm else 2,
                                     scaling=float(z[f"{nm}/scaling"]))
        np.testing.assert_array_equal(idx, z[f"{nm}/idx"], err_msg=nm)
        np.testing.assert_allclose(wt.astype(np.float32), _f16(z[f"{nm}/wts"]).astype(np.float32),
                                   atol=1e-3, rtol=0, err_msg=nm)


def test_grouped_router_planted_mistakes_fail():
    """Plausible mistakes in the group step each change a fixture: the group
    score as a sum instead of the max, the groups ignored, normalising when
    the config says not to."""
    z, names = _grouped_cases()

    def route(nm, group_score, use_groups, norm_override=None):
        E, k, ng, tg, norm = (int(v) for v in z[f"{nm}/cfg"])
        h = torch.from_numpy(_f16(z[f"{nm}/h"]).reshape(-1, 256)).float()
        s = torch.sigmoid(h @ torch.from_numpy(z[f"{nm}/w"]).t())
        if use_groups and ng > 1:
            g = s.view(-1, ng, E // ng)
            top = group_score(g).topk(tg, dim=-1).indices
            m = torch.zeros_like(g).scatter_(1, top.unsqueeze(-1).expand(-1, -1, E // ng), 1.0)
            s = (g * m).view(-1, E)
        tw, ti = s.topk(k, dim=-1)
        if (bool(norm) if norm_override is None else norm_override):
            tw = tw / (tw.sum(-1, keepdim=True) + 1e-9)
        return ti.numpy(), (tw * float(z[f"{nm}/scaling"])).half().numpy().view(np.uint16)

    grouped = [nm for nm in names if int(z[f"{nm}/cfg"][2]) > 1]
    for nm in grouped:
        ti, _ = route(nm, lambda g: g.sum(-1), True)
        assert not np.array_equal(ti, z[f"{nm}/idx"]), nm
        ti, _ = route(nm, lambda g: g.max(-1).values, False)
        assert not np.array_equal(ti, z[f"{nm}/idx"]), nm
        ti, tw = route(nm, lambda g: g.max(-1).values, True)
        assert np.array_equal(ti, z[f"{nm}/idx"]) and np.array_equal(tw, z[f"{nm}/wts"]), nm
    unnorm = [nm for nm in names if int(z[f"{nm}/cfg"][4]) == 0]
    assert unnorm
    for nm in unnorm:
        _, tw = route(nm, lambda g: g.max(-1).values, True, norm_override=True)
        assert not np.array_equal(tw, z[f"{nm}/wts"]), nm


def test_sigmoid_bias_selection_brute_force():
    rng = np.random.default_rng(9)
    T, E, k = 16, 32, 4
    lg = rng.standard_normal((T, E)).astype(np.float32)
    bias = rng.uniform(-0.1, 0.1, E).astype(np.float32)
    idx, w = oracle.router_topk(lg, k, mode=1, bias=bias)
    s = 1.0 / (1.0 + np.exp(-lg.astype(np.float64)))
    key = s.astype(np.float32) + bias
    for t in range(T):
        order = sorted(range(E), key=lambda e: (-key[t, e], e))[:k]
        assert list(idx[t]) == order
        ws = s[t, order]
        np.testing.assert_allclose(w[t].astype(np.float64), ws / ws.sum(), atol=1e-3)


# --------------------------------------------------------------------------- permute
@pytest.mark.parametrize("T,k,E", [(1, 2, 8), (4, 2, 8), (16, 2, 8), (32, 8, 128), (0, 2, 8),
                                   (300, 2, 8)])
def test_permute_brute_force(T, k, E):
    rng = np.random.default_rng(T * 31 + k)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32) \
        if T else np.zeros((0, k), np.int32)
    offsets, perm, inv, active = oracle.moe_permute(idx, E)
    flat = idx.reshape(-1)
    expect = sorted(range(flat.size), key=lambda j: (flat[j], j))
    assert list(perm) == expect
    assert all(perm[inv[j]] == j for j in range(flat.size))
    counts = np.bincount(flat, minlength=E)
    assert list(offsets) == [0] + list(np.cumsum(counts))
    assert list(active) == [e for e in range(E) if counts[e] > 0]


def test_unpermute_matches_index_add_fp16():
    rng = np.random.default_rng(3)
    T, k, E, H = 6, 2, 8, 16
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    w = rng.uniform(0, 1, (T, k)).astype(np.float16)
    offsets, perm, inv, active = oracle.moe_permute(idx, E)
    y = rng.standard_normal((T * k, H)).astype(np.float16)
    got = oracle.moe_unpermute(y, inv, idx, w)
    # reference: zeros fp16, per expert ascending: index_add_(0, tok, y_e * w)
    out = torch.zeros(T, H, dtype=torch.float16)
    ti = torch.from_numpy(idx.astype(np.int64))
    for e in active:
        tok, kp = torch.where(ti == int(e))
        rows = torch.from_numpy(y[[inv[t * k + s] for t, s in zip(tok.tolist(), kp.tolist())]])
        out.index_add_(0, tok, rows * torch.from_numpy(w)[tok, kp].unsqueeze(-1))
    assert np.array_equal(got.view(np.uint16), out.numpy().view(np.uint16))


def test_f16_conversion_matches_numpy_exhaustive_sample():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(200000).astype(np.float32) * s
                        for s in (1e-8, 1e-5, 1.0, 1e3, 7e4)])
    np.testing.assert_array_equal(oracle.f32_to_f16_bits(x), x.astype(np.float16).view(np.uint16))


# --------------------------------------------------------------------------- layout
def test_blob_layout_matches_reference_golden():
    from hydranet_amd.cache.blob_layout import BlobLayout
    with open(os.path.join(GOLD, "blob_layout.json")) as f:
        lay = json.load(f)
    for name, ent in lay.items():
        L = BlobLayout.from_dims(*ent["dims"])
        for field, v in ent.items():
            if field == "dims":
                continue
            assert getattr(L, field) == v, (name, field)
    # reference test_int4_pack.py:205-221 identities at 4096/14336/128
    L = BlobLayout.from_dims(4096, 14336, 128)
    assert L.total_size == 90832896


# --------------------------------------------------------------------------- MoE layers
def _gen():
    import importlib
    import sys
    if GOLD not in sys.path:
        sys.path.insert(0, GOLD)
    return importlib.import_module("gen")


def _seeded_experts(case_seed, E, H, I, g, digests=None, layer=0):
    """Regenerate the fixture's experts (tests/golden/gen.py) and pack them with
    the oracle packer; digests: the SHA-256 of the reference packer's bytes."""
    import hashlib
    gen = _gen()
    experts = {}
    for e in range(E):
        w = gen.expert_weights(case_seed, e, H, I, layer)
        parts = []
        for name in ("gate_proj", "up_proj", "down_proj"):
            p, s = oracle.quantize(w[name], g, mode=0)
            parts += [p, s]
        if digests is not None:
            h = hashlib.sha256()
            for a in parts:
                h.update(np.ascontiguousarray(a).tobytes())
            assert h.hexdigest() == str(digests[e]), f"expert {e}: packed bytes differ"
        experts[e] = tuple(torch.from_numpy(np.ascontiguousarray(a)) for a in parts)
    return experts


def _mixtral_fixture():
    z = _npz("mixtral_moe_layer.npz")
    H, I, g, E, seed = (int(v) for v in z["dims"])
    experts = _seeded_experts(seed, E, H, I, g, [z[f"sha/{e}"] for e in range(E)])
    h = torch.from_numpy(_f16(z["h"]).copy()).reshape(-1, H)
    gate = torch.from_numpy(_f16(z["gate"]).copy())
    return z, h, gate, experts, g


def test_torch_ref_mixtral_layer_matches_reference_layer():
    """torch_ref.mixtral_router / mixtral_moe / moe_dispatch against
    MixtralMoELayer.forward run by the reference (model/mixtral.py:259-370)."""
    z, h, gate, experts, g = _mixtral_fixture()
    for k in (2, 1):
        idx, w, logits = torch_ref.mixtral_router(h, gate, k)
        assert torch.equal(logits, torch.from_numpy(z[f"k{k}/logits"]).reshape(logits.shape))
        np.testing.assert_array_equal(idx.numpy(), z[f"k{k}/idx"].reshape(-1, k))
        np.testing.assert_array_equal(w.view(torch.int16).numpy().view(np.uint16),
                                      z[f"k{k}/w"].reshape(-1, k))
        y = torch_ref.mixtral_moe(h, gate, experts, top_k=k, group_size=g)
        np.testing.assert_array_equal(y.view(torch.int16).numpy().view(np.uint16),
                                      z[f"k{k}/out"].reshape(y.shape), err_msg=f"top-{k}")


def test_moe_dispatch_brute_force_per_token():
    """out[t] = sum over the token's experts in ascending id of fp16(fp16(y_e[t]) * w),
    accumulated in fp16 from zero, each y_e computed on the single row x_t."""
    z, h, gate, experts, g = _mixtral_fixture()
    for k in (2, 1):
        idx, w, _ = torch_ref.mixtral_router(h, gate, k)
        got = torch_ref.moe_dispatch(h, idx, w, experts, g)
        T, H = h.shape
        for t in range(T):
            acc = torch.zeros(H, dtype=torch.float16)
            for s in sorted(range(k), key=lambda s: int(idx[t, s])):
                y = torch_ref.expert_mlp(h[t:t + 1], *experts[int(idx[t, s])], group_size=g)[0]
                acc = acc + y * w[t, s]
            np.testing.assert_allclose(got[t].float().numpy(), acc.float().numpy(),
                                       atol=1e-3, rtol=1e-3)
        # the fixture's rows route tokens to distinct experts, so the ascending
        # order matters only through the fp16 sum; a wrong weight slot does not pass
        bad = torch_ref.moe_dispatch(h, idx, w.flip(-1), experts, g)
        if k > 1:
            assert not torch.equal(bad, got)


def _glm_fixture():
    z = _npz("glm_moe_layer.npz")
    H, I, g, E, k, seed = (int(v) for v in z["dims"])
    experts = _seeded_experts(seed, E, H, I, g, [z[f"sha/{e}"] for e in range(E)])
    sh = _gen().expert_weights(seed, 999, H, I)
    shared = tuple(torch.from_numpy(sh[n]) for n in ("gate_proj", "up_proj", "down_proj"))
    h = torch.from_numpy(_f16(z["h"]).copy()).reshape(-1, H)
    rw = torch.from_numpy(z["router_w"])
    return z, h, rw, experts, shared, k, g


def test_torch_ref_glm_layer_matches_reference_layer():
    """torch_ref.glm_router / glm_moe / dense_mlp against GLM4MoELayer.forward
    (model/glm4.py:365-473) with its fp16 shared expert, run by the reference."""
    z, h, rw, experts, shared, k, g = _glm_fixture()
    idx, w, _ = torch_ref.glm_router(h, rw, k)
    np.testing.assert_array_equal(idx.numpy(), z["idx"])
    np.testing.assert_array_equal(w.view(torch.int16).numpy().view(np.uint16), z["w"])
    y = torch_ref.glm_moe(h, rw, experts, shared, top_k=k, group_size=g)
    np.testing.assert_array_equal(y.view(torch.int16).numpy().view(np.uint16),
                                  z["out"].reshape(y.shape))
    # the selected-experts record used for next-layer prefetch (model/glm4.py:469)
    assert sorted(set(idx.reshape(-1).tolist())) == z["last_selected"].tolist()


def test_glm_dense_mlp_brute_force():
    """dense_mlp: SwiGLU of fp16 Linears, checked against float64 on the same weights."""
    z, h, rw, experts, shared, k, g = _glm_fixture()
    got = torch_ref.dense_mlp(h, *shared).double()
    gw, uw, dw = (t.double() for t in shared)
    x = h.double()
    a = x @ gw.t()
    ref = ((a * torch.sigmoid(a)) * (x @ uw.t())) @ dw.t()
    np.testing.assert_allclose(got.numpy(), ref.numpy(), atol=2e-3, rtol=1e-2)


def _dispatch_variant(h, idx, w, experts, g, order=sorted, fp32=False, init=None):
    out = torch.zeros(h.shape, dtype=torch.float32 if fp32 else torch.float16) \
        if init is None else init.clone()
    for e in order(idx.unique().tolist()):
        tok, kp = torch.where(idx == e)
        y = torch_ref.expert_mlp(h[tok], *experts[e], group_size=g)
        yw = y.float() * w[tok, kp].float().unsqueeze(-1) if fp32 else y * w[tok, kp].unsqueeze(-1)
        out.index_add_(0, tok, yw)
    return out.half()


def test_planted_layer_mistakes_are_caught():
    """Plausible slips in the dispatch restatement fail the layer fixtures:
    fp32 accumulation (Mixtral top-2), descending expert order and the shared
    expert used as the accumulator's start (GLM top-4)."""
    z, h, gate, experts, g = _mixtral_fixture()
    idx, w, _ = torch_ref.mixtral_router(h, gate, 2)
    bad = _dispatch_variant(h, idx, w, experts, g, fp32=True)
    assert not np.array_equal(bad.view(torch.int16).numpy().view(np.uint16),
                              z["k2/out"].reshape(bad.shape))
    z, h, rw, experts, shared, k, g = _glm_fixture()
    idx, w, _ = torch_ref.glm_router(h, rw, k)
    ref = z["out"].reshape(h.shape)
    sh = torch_ref.dense_mlp(h, *shared)
    desc = sh + _dispatch_variant(h, idx, w, experts, g,
                                  order=lambda v: sorted(v, reverse=True))
    first = _dispatch_variant(h, idx, w, experts, g, init=sh)
    for bad in (desc, first):
        assert not np.array_equal(bad.view(torch.int16).numpy().view(np.uint16), ref)


def test_affinity_bonus_matches_reference_golden():
    """TopKRouter.forward with the cache-affinity bonus on (model/router.py:96-175),
    experts 1, 4, 6 cached: logits, indices and weights bit for bit; the
    build's TopKRouter._affinity (host torch ops) equals it too."""
    from hydranet_amd.model.router import TopKRouter
    z = _npz("affinity_router.npz")
    h = torch.from_numpy(_f16(z["h"]).copy()).reshape(-1, 256)
    gate = torch.from_numpy(_f16(z["gate"]).copy())
    cached = z["cached"].tolist()
    bonus, thr = (float(v) for v in z["bonus"])
    raw = torch.nn.functional.linear(h, gate).float()
    gated = 0
    for k in (1, 2):
        idx, w, logits = torch_ref.mixtral_router(h, gate, k, cached=cached, bonus=bonus,
                                                  threshold=thr)
        ref_lg = torch.from_numpy(z[f"k{k}/logits"]).reshape(logits.shape)
        assert torch.equal(logits, ref_lg)
        np.testing.assert_array_equal(idx.numpy(), z[f"k{k}/idx"].reshape(-1, k))
        np.testing.assert_array_equal(w.view(torch.int16).numpy().view(np.uint16),
                                      z[f"k{k}/w"].reshape(-1, k))
        gated = int((logits != raw).any(-1).sum())
        r = TopKRouter(256, 8, 2, affinity_bonus=bonus, entropy_threshold=thr,
                       enable_affinity_bonus=True)
        r.set_cache_checker(lambda e: e in cached)
        assert torch.equal(r._affinity(raw), ref_lg)
    # the fixture has tokens on both sides of the entropy threshold
    assert 0 < gated < h.shape[0]
